"""Flow front-end on libfcvdit.so: speech tokens, prompt Mel and x-vectors -> packed mu/cond/spks,
then the packed CFG solve; mirrors ``flow_inference_batched`` and
``flow_inference_batched_streaming`` (faster_cosyvoice/token2wav/flashinfer_flow.py:118-184,
207-281).

``FlowFrontEnd`` holds the front-end parameters under the reference's module names
(``input_embedding``, ``pre_lookahead_layer.conv1/conv2``, ``spk_embed_affine_layer``,
cosyvoice/flow/flow.py:307-313), so ``load_reference_state_dict`` takes a ``flow.pt`` state
dict as it is.  All compute runs in libfcvdit.so (include/fcv_flow.h), in fp32.
"""

from __future__ import annotations

from collections.abc import Sequence
from typing import Any

import torch
import torch.nn as nn

from . import _lib
from .estimator import DiTEstimator
from .solver import solve_euler_packed

_PREFIXES = ("input_embedding.", "spk_embed_affine_layer.", "pre_lookahead_layer.")


class _PreLookaheadParams(nn.Module):
    """Parameters of ``PreLookaheadLayer`` (upsample_encoder.py:55-70)."""

    def __init__(self, in_channels: int, channels: int, pre_lookahead_len: int, device):
        super().__init__()
        self.pre_lookahead_len = pre_lookahead_len
        self.conv1 = nn.Conv1d(in_channels, channels, pre_lookahead_len + 1, device=device)
        self.conv2 = nn.Conv1d(channels, in_channels, 3, device=device)


class FlowFrontEnd(nn.Module):
    """Token embedding + PreLookaheadLayer + speaker projection of ``CausalMaskedDiffWithDiT``
    (builders.py:29-35 shapes by default)."""

    def __init__(self, vocab_size: int = 6561, input_size: int = 80, output_size: int = 80,
                 spk_embed_dim: int = 192, channels: int = 1024, pre_lookahead_len: int = 3,
                 token_mel_ratio: int = 2, device: torch.device | str = "cuda:0"):
        super().__init__()
        if input_size != output_size:
            raise ValueError("input_size must equal output_size (mu and the Mel share channels)")
        self.device = torch.device(device)
        self.output_size = output_size
        self.token_mel_ratio = token_mel_ratio
        self.pre_lookahead_len = pre_lookahead_len
        self.input_embedding = nn.Embedding(vocab_size, input_size, device=device)
        self.spk_embed_affine_layer = nn.Linear(spk_embed_dim, output_size, device=device)
        self.pre_lookahead_layer = _PreLookaheadParams(input_size, channels, pre_lookahead_len,
                                                       device)
        self.dims = _lib.FcvFlowDims(vocab=vocab_size, feat_dim=input_size, channels=channels,
                                     lookahead=pre_lookahead_len, token_mel_ratio=token_mel_ratio,
                                     spk_dim=spk_embed_dim)
        self._derived: dict[str, torch.Tensor] | None = None
        self._weights: _lib.FcvFlowWeights | None = None
        self._ws: torch.Tensor | None = None
        self._lib = _lib.load()

    # ---- construction ----------------------------------------------------------------------

    @classmethod
    def from_flow(cls, flow: Any, device: torch.device | str | None = None) -> "FlowFrontEnd":
        """Front-end with the shapes and weights of a reference ``CausalMaskedDiffWithDiT``."""
        emb = flow.input_embedding.weight
        la = flow.pre_lookahead_layer
        fe = cls(vocab_size=emb.shape[0], input_size=emb.shape[1], output_size=flow.output_size,
                 spk_embed_dim=flow.spk_embed_affine_layer.weight.shape[1],
                 channels=la.conv1.weight.shape[0], pre_lookahead_len=flow.pre_lookahead_len,
                 token_mel_ratio=flow.token_mel_ratio,
                 device=device if device is not None else emb.device)
        fe.load_reference_state_dict(flow.state_dict())
        fe.finalize_weights()
        return fe

    def load_reference_state_dict(self, sd: dict[str, torch.Tensor]) -> None:
        """Load the front-end entries of a flow state dict (other keys are ignored)."""
        own = {k: v for k, v in sd.items() if k.startswith(_PREFIXES)}
        self.load_state_dict({k: v.float() for k, v in own.items()}, strict=True)
        self._derived = None

    @torch.no_grad()
    def finalize_weights(self) -> None:
        """fp32 device copies in the kernels' layouts: convolution weights tap-major, so
        ``la1_w[c][tap*F + i] = conv1.weight[c][i][tap]``, ``la2_w[o][tap*C + c] =
        conv2.weight[o][c][tap]``."""
        dev = self.device
        f32 = lambda t: t.detach().to(device=dev, dtype=torch.float32).contiguous()
        w1 = self.pre_lookahead_layer.conv1.weight
        w2 = self.pre_lookahead_layer.conv2.weight
        d = {
            "embed": f32(self.input_embedding.weight),
            "la1_w": f32(w1.permute(0, 2, 1).reshape(w1.shape[0], -1)),
            "la1_b": f32(self.pre_lookahead_layer.conv1.bias),
            "la2_w": f32(w2.permute(0, 2, 1).reshape(w2.shape[0], -1)),
            "la2_b": f32(self.pre_lookahead_layer.conv2.bias),
            "spk_w": f32(self.spk_embed_affine_layer.weight),
            "spk_b": f32(self.spk_embed_affine_layer.bias),
        }
        self._derived = d
        self._weights = _lib.FcvFlowWeights(**{k: v.data_ptr() for k, v in d.items()})

    def _require(self) -> _lib.FcvFlowWeights:
        if self._weights is None:
            raise RuntimeError("call finalize_weights() before running the front-end")
        return self._weights

    def _workspace(self, out_tokens: int) -> torch.Tensor:
        need = int(self._lib.fcv_flow_workspace_bytes(self.dims, out_tokens))
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.device)
        return self._ws

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    # ---- the three front-end operations ----------------------------------------------------

    @torch.no_grad()
    def token_features(self, token_list: Sequence[Sequence[int]],
                       finalize_list: Sequence[bool] | None = None
                       ) -> tuple[torch.Tensor, list[int]]:
        """Packed mu rows ``[sum(mel_lengths), 80]`` and the per-document Mel lengths.

        ``finalize_list`` None: every document is complete (flashinfer_flow.py:148-151, the
        offline path); False for a document: its last ``pre_lookahead_len`` tokens are right
        context only (``_streaming_token_features``, flashinfer_flow.py:187-204)."""
        if len(token_list) == 0:
            raise ValueError("token_list is empty")
        lengths = [len(t) for t in token_list]
        flat = [int(v) for t in token_list for v in t]
        vocab = self.dims.vocab
        if flat and max(flat) >= vocab:
            raise IndexError("index out of range in self")  # nn.Embedding's error
        if finalize_list is not None and len(finalize_list) != len(lengths):
            raise ValueError("token_list and finalize_list must have the same length")
        tokens = torch.tensor(flat, dtype=torch.int32).to(self.device)
        return self.token_features_device(tokens, lengths, finalize_list)

    @torch.no_grad()
    def token_features_device(self, tokens: torch.Tensor, lengths: Sequence[int],
                              finalize_list: Sequence[bool] | None = None,
                              out: torch.Tensor | None = None) -> tuple[torch.Tensor, list[int]]:
        """``token_features`` on device-resident packed int32 ids (document d owns
        ``lengths[d]`` consecutive ids); asynchronous on the current stream.  Ids >= vocab are
        not checked here and read the last embedding row.  ``out``: optional preallocated
        ``[>= rows, 80]`` fp32 buffer."""
        lengths = [int(n) for n in lengths]
        L, ratio = self.pre_lookahead_len, self.token_mel_ratio
        fin = [True] * len(lengths) if finalize_list is None else [bool(f) for f in finalize_list]
        if len(fin) != len(lengths):
            raise ValueError("token_list and finalize_list must have the same length")
        if tokens.dtype != torch.int32 or tokens.device != self.device or tokens.dim() != 1:
            raise ValueError("tokens must be a 1-D int32 tensor on the front-end's device")
        if tokens.numel() != sum(lengths):
            raise ValueError(f"tokens holds {tokens.numel()} ids, lengths sum to {sum(lengths)}")
        tokens = tokens.contiguous()
        out_tokens = [n - (0 if f else L) for n, f in zip(lengths, fin)]
        rows = ratio * max(sum(out_tokens), 0)
        if out is None:
            out = torch.empty(max(rows, 1), self.output_size, dtype=torch.float32,
                              device=self.device)
        elif (out.dtype != torch.float32 or out.device != self.device or not out.is_contiguous()
              or out.shape[0] < rows or out.shape[1] != self.output_size):
            raise ValueError(f"out must be a contiguous fp32 [>= {rows}, {self.output_size}] "
                             "tensor on the front-end's device")
        # one library call per group of at most FLOW_MAX_DOCS documents; a document's rows do
        # not depend on its group
        groups = [slice(g0, g0 + _lib.FLOW_MAX_DOCS)
                  for g0 in range(0, len(lengths), _lib.FLOW_MAX_DOCS)]
        ws = self._workspace(max(max(sum(out_tokens[g]), 0) for g in groups))
        tok_off = row_off = 0
        for g in groups:
            cu = [0]
            for n in lengths[g]:
                cu.append(cu[-1] + n)
            _lib.check(self._lib.fcv_flow_token_features(
                self.dims, self._require(), tokens.data_ptr() + 4 * tok_off,
                (_lib.c_int32 * len(cu))(*cu),
                (_lib.c_int32 * len(fin[g]))(*[int(f) for f in fin[g]]), len(cu) - 1,
                out.data_ptr() + 4 * self.output_size * row_off, ws.data_ptr(), ws.numel(),
                self._stream()))
            tok_off += cu[-1]
            row_off += ratio * sum(out_tokens[g])
        return out[:rows], [ratio * n for n in out_tokens]

    @torch.no_grad()
    def speaker(self, speaker_embeddings: torch.Tensor) -> torch.Tensor:
        """``spk_embed_affine_layer(F.normalize(x, dim=1))`` (flashinfer_flow.py:145-146)."""
        x = speaker_embeddings.to(device=self.device, dtype=torch.float32).contiguous()
        if x.dim() != 2 or x.shape[1] != self.dims.spk_dim:
            raise ValueError(f"speaker_embeddings must be [B, {self.dims.spk_dim}]")
        out = torch.empty(x.shape[0], self.output_size, dtype=torch.float32, device=self.device)
        _lib.check(self._lib.fcv_flow_speaker(self.dims, self._require(), x.data_ptr(),
                                              x.shape[0], out.data_ptr(), self._stream()))
        return out

    @torch.no_grad()
    def prompt_condition(self, prompt_features: Sequence[torch.Tensor],
                         mel_lengths: Sequence[int]) -> tuple[torch.Tensor, list[int]]:
        """Packed condition rows: each document's prompt Mel ``(1, P, 80)`` in its first
        frames, zeros after (``_copy_prompt_features``, flashinfer_flow.py:93-115)."""
        if len(prompt_features) != len(mel_lengths):
            raise ValueError("one prompt per document is required")
        max_mel = max(mel_lengths)
        plens = [int(p.shape[1]) for p in prompt_features]
        for p in prompt_features:
            if p.dim() != 3 or p.shape[0] != 1 or p.shape[2] != self.output_size:
                raise ValueError(f"prompt features must be (1, P, {self.output_size})")
            if p.shape[1] > max_mel:  # the reference's padded copy cannot hold it either
                raise RuntimeError(f"prompt of {p.shape[1]} frames exceeds the longest "
                                   f"document ({max_mel} frames)")
        prompt = (torch.cat([p[0] for p in prompt_features]) if sum(plens) else
                  torch.zeros(1, self.output_size))
        prompt = prompt.to(device=self.device, dtype=torch.float32).contiguous()
        cu_p, cu_m = [0], [0]
        for p, m in zip(plens, mel_lengths):
            cu_p.append(cu_p[-1] + p)
            cu_m.append(cu_m[-1] + int(m))
        cond = torch.empty(cu_m[-1], self.output_size, dtype=torch.float32, device=self.device)
        for g0 in range(0, len(plens), _lib.FLOW_MAX_DOCS):
            g1 = min(g0 + _lib.FLOW_MAX_DOCS, len(plens))
            cp = [v - cu_p[g0] for v in cu_p[g0:g1 + 1]]
            cm = [v - cu_m[g0] for v in cu_m[g0:g1 + 1]]
            _lib.check(self._lib.fcv_flow_prompt_cond(
                self.dims, prompt.data_ptr() + 4 * self.output_size * cu_p[g0],
                (_lib.c_int32 * len(cp))(*cp), (_lib.c_int32 * len(cm))(*cm), g1 - g0,
                cond.data_ptr() + 4 * self.output_size * cu_m[g0], self._stream()))
        return cond, plens


def frontend_for(flow: Any) -> FlowFrontEnd:
    """The ``FlowFrontEnd`` serving ``flow``: ``flow`` itself, or one built from its modules
    once and cached on it."""
    if isinstance(flow, FlowFrontEnd):
        return flow
    fe = getattr(flow, "_mi355x_frontend", None)
    if fe is None:
        fe = FlowFrontEnd.from_flow(flow)
        flow._mi355x_frontend = fe
    return fe


def _decoder_estimator(flow: Any) -> DiTEstimator:
    est = flow.decoder.estimator
    if not isinstance(est, DiTEstimator):
        raise TypeError("flow.decoder.estimator must be a DiTEstimator (see apply_mi355x)")
    return est


def _pack_noise(noise: torch.Tensor, mel_lengths: Sequence[int]) -> torch.Tensor:
    return torch.cat([noise[b, :, :n].transpose(0, 1) for b, n in enumerate(mel_lengths)])


def _split_generated(x: torch.Tensor, mel_lengths: Sequence[int],
                     prompt_lengths: Sequence[int]) -> list[torch.Tensor]:
    out, off = [], 0
    for n, p in zip(mel_lengths, prompt_lengths):
        out.append(x[off + min(p, n):off + n].transpose(0, 1).unsqueeze(0).float())
        off += n
    return out


@torch.no_grad()
def flow_inference_batched(flow: Any, token_list: Sequence[Sequence[int]],
                           prompt_features: Sequence[torch.Tensor],
                           speaker_embeddings: torch.Tensor, *,
                           noise: torch.Tensor | None = None) -> list[torch.Tensor]:
    """Offline Flow inference for variable-length samples (flashinfer_flow.py:118-184).

    ``flow``: a ``FlowFrontEnd`` carrying a ``decoder`` (``.estimator`` a ``DiTEstimator``,
    ``.inference_cfg_rate``), or a reference flow whose decoder estimator was replaced by
    ``apply_mi355x``.  Returns one ``(1, 80, mel_len - prompt_len)`` fp32 tensor per sample.
    ``noise`` (``[B, 80, max_mel]``) replaces the ``torch.randn`` draw when given."""
    fe = frontend_for(flow)
    est = _decoder_estimator(flow)
    mu, mel_lengths = fe.token_features(token_list)
    spks = fe.speaker(speaker_embeddings)
    cond, prompt_lengths = fe.prompt_condition(prompt_features, mel_lengths)
    max_mel = max(mel_lengths)
    if noise is None:
        noise = torch.randn(len(token_list), fe.output_size, max_mel, device=fe.device,
                            dtype=torch.float32)
    x = solve_euler_packed(est, _pack_noise(noise, mel_lengths), mu, cond, spks, mel_lengths,
                           n_steps=10, cfg_rate=float(flow.decoder.inference_cfg_rate),
                           streaming=False)
    return _split_generated(x, mel_lengths, prompt_lengths)


@torch.no_grad()
def flow_inference_batched_streaming(flow: Any, token_list: Sequence[Sequence[int]],
                                     prompt_features: Sequence[torch.Tensor],
                                     speaker_embeddings: torch.Tensor,
                                     finalize_list: Sequence[bool]) -> list[torch.Tensor]:
    """Full-prefix streaming Flow inference for several streams (flashinfer_flow.py:207-281):
    non-final streams keep their last ``pre_lookahead_len`` tokens as lookahead context, every
    stream starts from the decoder's fixed noise prefix, chunk-causal attention."""
    if len(token_list) != len(finalize_list):
        raise ValueError("token_list and finalize_list must have the same length")
    fe = frontend_for(flow)
    est = _decoder_estimator(flow)
    spks = fe.speaker(speaker_embeddings)
    mu, mel_lengths = fe.token_features(token_list, finalize_list)
    cond, prompt_lengths = fe.prompt_condition(prompt_features, mel_lengths)
    rand = flow.decoder.rand_noise
    max_mel = max(mel_lengths)
    if rand.shape[-1] < max_mel:
        raise ValueError(f"decoder.rand_noise holds {rand.shape[-1]} frames, need {max_mel}")
    prefix = rand[0, :, :max_mel].to(device=fe.device, dtype=torch.float32)
    noise = torch.cat([prefix[:, :n].transpose(0, 1) for n in mel_lengths])
    x = solve_euler_packed(est, noise, mu, cond, spks, mel_lengths, n_steps=10,
                           cfg_rate=float(flow.decoder.inference_cfg_rate), streaming=True)
    return _split_generated(x, mel_lengths, prompt_lengths)
