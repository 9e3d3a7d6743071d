"""fp32 CPU restatement of the Flow front-end that produces the DiT inputs mu / cond / spks.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Paths are relative to the reference root
``faster_cosyvoice/token2wav/``.

* token embedding with clamped ids, zeroed past each sequence:
  ``flashinfer_flow.py:144-149`` (``flow.input_embedding(torch.clamp(tokens, min=0)) * mask``);
* ``PreLookaheadLayer`` (``cosyvoice/transformer/upsample_encoder.py:55-92``): right zero pad of
  ``pre_lookahead_len`` frames (or the lookahead context), conv1 (kernel lookahead + 1),
  LeakyReLU (slope 0.01), causal left pad of 2 frames, conv2 (kernel 3), residual;
* ``repeat_interleave(token_mel_ratio)`` to mel frames (``flashinfer_flow.py:150``);
* speaker path ``F.normalize(x, dim=1)`` then ``spk_embed_affine_layer`` (``:145-146``);
* prompt Mel copied into the first frames of ``cond`` (``_copy_prompt_features``, ``:92-115``);
* streaming token features with a right context (``_streaming_token_features``, ``:210-227``).
"""

from __future__ import annotations

from typing import Mapping, Sequence

import torch
import torch.nn.functional as F

Tensor = torch.Tensor


def embed_tokens(table: Tensor, tokens: Tensor, lengths: Sequence[int]) -> Tensor:
    """``input_embedding(clamp(tokens, 0)) * mask``: ``tokens`` [B, T] -> [B, T, C]."""
    x = table[torch.clamp(tokens, min=0)]
    mask = torch.zeros(tokens.shape, dtype=x.dtype)
    for b, n in enumerate(lengths):
        mask[b, :n] = 1.0
    return x * mask.unsqueeze(-1)


def pre_lookahead(x: Tensor, w1: Tensor, b1: Tensor, w2: Tensor, b2: Tensor, lookahead: int = 3,
                  context: Tensor | None = None) -> Tensor:
    """``PreLookaheadLayer.forward`` (upsample_encoder.py:72-92) on ``x`` [B, T, C]."""
    out = x.transpose(1, 2)
    if context is None or context.shape[1] == 0:
        out = F.pad(out, (0, lookahead))
    else:
        out = F.pad(torch.cat([out, context.transpose(1, 2)], dim=2),
                    (0, lookahead - context.shape[1]))
    out = F.leaky_relu(F.conv1d(out, w1, b1))
    out = F.pad(out, (w2.shape[2] - 1, 0))
    out = F.conv1d(out, w2, b2).transpose(1, 2)
    return out + x


def speaker_projection(xvec: Tensor, w: Tensor, b: Tensor) -> Tensor:
    """``spk_embed_affine_layer(F.normalize(xvec, dim=1))``: [B, 192] -> [B, 80]."""
    return F.linear(F.normalize(xvec, dim=1), w, b)


def flow_inputs(sd: Mapping[str, Tensor], token_list: Sequence[Sequence[int]],
                prompt_features: Sequence[Tensor], xvec: Tensor, token_mel_ratio: int = 2,
                lookahead: int = 3):
    """The estimator inputs ``flow_inference_batched`` builds (flashinfer_flow.py:141-161):
    returns mu [B, 80, Tm], cond [B, 80, Tm], spks [B, 80], mel lengths, prompt lengths."""
    lengths = [len(t) for t in token_list]
    tokens = torch.zeros(len(token_list), max(lengths), dtype=torch.long)
    for b, t in enumerate(token_list):
        tokens[b, :len(t)] = torch.tensor(list(t), dtype=torch.long)
    spks = speaker_projection(xvec.float(), sd["spk_embed_affine_layer.weight"],
                              sd["spk_embed_affine_layer.bias"])
    feats = embed_tokens(sd["input_embedding.weight"], tokens, lengths)
    mu = pre_lookahead(feats, sd["pre_lookahead_layer.conv1.weight"],
                       sd["pre_lookahead_layer.conv1.bias"], sd["pre_lookahead_layer.conv2.weight"],
                       sd["pre_lookahead_layer.conv2.bias"], lookahead)
    mu = mu.repeat_interleave(token_mel_ratio, dim=1)
    mel_lengths = [n * token_mel_ratio for n in lengths]
    tm = max(mel_lengths)
    cond = torch.zeros(len(token_list), tm, mu.shape[-1])
    prompt_lengths = []
    for b, p in enumerate(prompt_features):
        prompt_lengths.append(p.shape[1])
        cond[b, :p.shape[1]] = p[0].float()
    return mu.transpose(1, 2), cond.transpose(1, 2), spks, mel_lengths, prompt_lengths


def streaming_token_features(sd: Mapping[str, Tensor], tokens: Sequence[int], finalize: bool,
                             token_mel_ratio: int = 2, lookahead: int = 3) -> Tensor:
    """``_streaming_token_features`` (flashinfer_flow.py:210-227): one stream's mu rows; when
    not finalizing, the last ``lookahead`` tokens only serve as right context."""
    t = torch.tensor([list(tokens)], dtype=torch.long)
    emb = sd["input_embedding.weight"][torch.clamp(t, min=0)]
    w = [sd[f"pre_lookahead_layer.{k}"] for k in ("conv1.weight", "conv1.bias", "conv2.weight",
                                                  "conv2.bias")]
    if finalize:
        feats = pre_lookahead(emb, *w, lookahead)
    else:
        feats = pre_lookahead(emb[:, :-lookahead], *w, lookahead, context=emb[:, -lookahead:])
    return feats.repeat_interleave(token_mel_ratio, dim=1)
