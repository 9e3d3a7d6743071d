"""The on-disk Flow format: a ``flow.pt`` state dict -> the MI355X flow (front-end + packed DiT
estimator + CFG decoder attributes).

The reference builds ``CausalMaskedDiffWithDiT`` (builders.py:16-35), loads ``flow.pt`` into it
with ``strict=True`` (token2wav.py:66-69), then swaps the estimator and derives its inference
weights (``apply_flashinfer``, flashinfer_dit.py:951-988).  ``load_flow`` does the same from the
state dict alone: it splits the keys into the front-end (``input_embedding``,
``spk_embed_affine_layer``, ``pre_lookahead_layer``) and the estimator
(``decoder.estimator.*``), reads every shape from the tensors, and rejects any other key, as
the strict load does.  The estimator's RoPE buffers are skipped, as in the reference
(flashinfer_dit.py:975-983).  Files are read with ``torch.load(weights_only=True)`` only.
"""

from __future__ import annotations

import re
from pathlib import Path
from typing import Mapping

import torch

from .estimator import DiTEstimator
from .frontend import _PREFIXES, FlowFrontEnd
from .streaming import CFMDecoder

ESTIMATOR_PREFIX = "decoder.estimator."


def split_flow_state_dict(sd: Mapping[str, torch.Tensor]
                          ) -> tuple[dict[str, torch.Tensor], dict[str, torch.Tensor]]:
    """(front-end entries, estimator entries without their ``decoder.estimator.`` prefix);
    ``RuntimeError`` for keys that belong to neither."""
    front = {k: v for k, v in sd.items() if k.startswith(_PREFIXES)}
    est = {k[len(ESTIMATOR_PREFIX):]: v for k, v in sd.items() if k.startswith(ESTIMATOR_PREFIX)}
    other = [k for k in sd if k not in front and not k.startswith(ESTIMATOR_PREFIX)]
    if other:
        raise RuntimeError(f"unexpected keys in the flow state dict: {other[:8]}")
    if not front or not est:
        raise RuntimeError("the flow state dict needs front-end and decoder.estimator entries")
    return front, est


def flow_shapes(front: Mapping[str, torch.Tensor], est: Mapping[str, torch.Tensor]) -> dict:
    """Every hyper-parameter ``load_flow`` needs, read from the tensors' shapes."""
    vocab, feat = front["input_embedding.weight"].shape
    channels, _, k1 = front["pre_lookahead_layer.conv1.weight"].shape
    spk_dim = front["spk_embed_affine_layer.weight"].shape[1]
    blocks = {int(m.group(1)) for k in est
              if (m := re.match(r"transformer_blocks\.(\d+)\.", k))}
    if not blocks or blocks != set(range(max(blocks) + 1)):
        raise RuntimeError("decoder.estimator.transformer_blocks.* are missing or not contiguous")
    mel, dim = est["proj_out.weight"].shape
    inner = est["transformer_blocks.0.attn.to_q.weight"].shape[0]
    ff_dim = est["transformer_blocks.0.ff.ff.0.0.weight"].shape[0]
    dim_head = 64
    if inner % dim_head or ff_dim % dim:
        raise RuntimeError(f"unsupported estimator shape: inner {inner}, ff {ff_dim}, dim {dim}")
    return dict(vocab=vocab, feat=feat, channels=channels, lookahead=k1 - 1, spk_dim=spk_dim,
                depth=max(blocks) + 1, dim=dim, heads=inner // dim_head, dim_head=dim_head,
                ff_mult=ff_dim // dim, mel=mel)


def load_flow(source: str | Path | Mapping[str, torch.Tensor], device: str = "cuda:0",
              static_chunk_size: int = 50, inference_cfg_rate: float = 0.7,
              token_mel_ratio: int = 2, noise_seed: int = 0) -> FlowFrontEnd:
    """Build the MI355X flow from ``flow.pt`` (a path, or its already-loaded state dict).

    Returns a ``FlowFrontEnd`` whose ``decoder`` is a ``CFMDecoder`` holding the finalized
    ``DiTEstimator``: the ``flow`` argument of ``flow_inference_batched[_streaming]`` and
    ``StreamingFlow``.  Defaults follow builders.py:17-35 (chunk 50, CFG 0.7, ratio 2); the
    fixed noise prefix is the reference's (seed 0, flow_matching.py:199-200)."""
    if isinstance(source, (str, Path)):
        sd = torch.load(str(source), map_location="cpu", weights_only=True)
    else:
        sd = dict(source)
    front, est_sd = split_flow_state_dict(sd)
    s = flow_shapes(front, est_sd)
    fe = FlowFrontEnd(vocab_size=s["vocab"], input_size=s["feat"], output_size=s["mel"],
                      spk_embed_dim=s["spk_dim"], channels=s["channels"],
                      pre_lookahead_len=s["lookahead"], token_mel_ratio=token_mel_ratio,
                      device=device)
    fe.load_reference_state_dict(front)
    fe.finalize_weights()
    est = DiTEstimator(dim=s["dim"], depth=s["depth"], heads=s["heads"], dim_head=s["dim_head"],
                       ff_mult=s["ff_mult"], mel_dim=s["mel"], mu_dim=s["mel"],
                       spk_dim=s["mel"], out_channels=s["mel"],
                       static_chunk_size=static_chunk_size, device=device)
    est.load_reference_state_dict(est_sd)
    est.finalize_weights()
    fe.decoder = CFMDecoder(est, inference_cfg_rate=inference_cfg_rate, noise_seed=noise_seed)
    return fe
