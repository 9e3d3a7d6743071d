"""fp32 CPU restatement of the CosyVoice3 DiT estimator and its CFG Euler solver.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Every function cites
the reference file:line it follows; paths are relative to the reference root
``faster_cosyvoice/token2wav/``.

Semantics restated here (the traps are called out where they occur):

* timestep embedding: ``cosyvoice/flow/DiT/modules.py:71-83,606-616``;
* input embedding + *causal* grouped conv position embedding:
  ``cosyvoice/flow/DiT/dit.py:76-98``, ``modules.py:115-144``;
* RoPE: x_transformers ``RotaryEmbedding(dim_head)`` applied to the *flat*
  1024-wide q/k before the head split (``modules.py:363-380``), so only flat
  columns ``0..dim_head-1`` (all of head 0) rotate, interleaved pairs
  ``(2i, 2i+1)``; the reference restates the same rotation in
  ``flashinfer_dit.py:262-273`` and ``flashinfer_kernels.py:219-249``;
* DiT block (AdaLN-Zero, SDPA with a boolean mask, tanh-GELU FFN):
  ``modules.py:230-244,271-282,349-407,500-530``;
* masks: ``cosyvoice/utils/mask.py:127-236`` called from ``dit.py:163-166``;
* final AdaLN ``(scale, shift)`` order: ``modules.py:251-265``;
* DiT forward: ``dit.py:145-176``;
* packed CFG Euler solver with the cosine schedule:
  ``flashinfer_flow.py:16-74`` (same arithmetic as
  ``cosyvoice/flow/flow_matching.py:71-124`` for one request).

Parity of the x_transformers RoPE arithmetic itself is pinned only through
the reference's two in-repo restatements and the rotation invariants tested
in ``tests/test_oracle.py`` (x_transformers 2.23.5 is not installed here).
"""

from __future__ import annotations

import math
from typing import Callable, Mapping, Sequence

import torch
import torch.nn.functional as F

Tensor = torch.Tensor
StateDict = Mapping[str, Tensor]

LN_EPS = 1e-6


# --------------------------------------------------------------------------
# small pieces


def sinus_position_embedding(t: Tensor, dim: int = 256, scale: float = 1000.0) -> Tensor:
    """``SinusPositionEmbedding.forward`` (modules.py:76-83)."""
    half = dim // 2
    step = math.log(10000) / (half - 1)
    freqs = torch.exp(torch.arange(half, dtype=torch.float32) * -step)
    arg = scale * t.float().unsqueeze(1) * freqs.unsqueeze(0)
    return torch.cat((arg.sin(), arg.cos()), dim=-1)


def timestep_embedding(sd: StateDict, t: Tensor) -> Tensor:
    """``TimestepEmbedding.forward`` (modules.py:606-616): sinusoid -> Linear -> SiLU -> Linear."""
    hidden = sinus_position_embedding(t)
    hidden = F.linear(hidden, sd["time_embed.time_mlp.0.weight"], sd["time_embed.time_mlp.0.bias"])
    hidden = F.silu(hidden)
    return F.linear(hidden, sd["time_embed.time_mlp.2.weight"], sd["time_embed.time_mlp.2.bias"])


def rotary_freqs(positions: Tensor, dim_head: int = 64, base: float = 10000.0) -> Tensor:
    """x_transformers ``RotaryEmbedding(dim_head).forward`` as used at dit.py:129,158.

    Returns ``[len(positions), dim_head]`` angles in the interleaved layout
    ``(d r)``: columns ``2i`` and ``2i+1`` share the angle ``p * base^(-2i/dim_head)``
    (the reference's table ``freqs[:, 0::2]``, flashinfer_dit.py:266-273).
    """
    inv_freq = 1.0 / (base ** (torch.arange(0, dim_head, 2, dtype=torch.float32) / dim_head))
    angles = positions.to(torch.float32)[:, None] * inv_freq[None, :]
    return torch.stack((angles, angles), dim=-1).reshape(positions.shape[0], dim_head)


def _rotate_half_interleaved(x: Tensor) -> Tensor:
    pairs = x.reshape(*x.shape[:-1], x.shape[-1] // 2, 2)
    even, odd = pairs.unbind(-1)
    return torch.stack((-odd, even), dim=-1).reshape(x.shape)


def apply_rotary(x: Tensor, freqs: Tensor) -> Tensor:
    """x_transformers ``apply_rotary_pos_emb`` on the flat projection (modules.py:368-373).

    ``x`` is ``[..., T, D]`` (D = heads*dim_head, not yet split); only the first
    ``freqs.shape[-1]`` columns rotate: ``(a, b) -> (a cos - b sin, b cos + a sin)``.
    """
    rot = freqs.shape[-1]
    head, rest = x[..., :rot], x[..., rot:]
    head = head * freqs.cos() + _rotate_half_interleaved(head) * freqs.sin()
    return torch.cat((head, rest), dim=-1)


def layer_norm(x: Tensor) -> Tensor:
    """``nn.LayerNorm(dim, elementwise_affine=False, eps=1e-6)`` (modules.py:237,513)."""
    mean = x.mean(-1, keepdim=True)
    var = ((x - mean) ** 2).mean(-1, keepdim=True)
    return (x - mean) / torch.sqrt(var + LN_EPS)


def gelu_tanh(x: Tensor) -> Tensor:
    """``nn.GELU(approximate="tanh")`` (modules.py:275)."""
    return 0.5 * x * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))


def mish(x: Tensor) -> Tensor:
    """``nn.Mish`` (modules.py:120-126): ``x * tanh(softplus(x))``."""
    return x * torch.tanh(F.softplus(x))


# --------------------------------------------------------------------------
# masks


def subsequent_chunk_mask(size: int, chunk_size: int) -> Tensor:
    """``subsequent_chunk_mask`` (mask.py:127-158): key k visible to query q iff k < (q//c + 1)*c."""
    pos = torch.arange(size)
    limit = (torch.div(pos, chunk_size, rounding_mode="trunc") + 1) * chunk_size
    return pos.unsqueeze(0) < limit.unsqueeze(1)


def attention_mask(mask: Tensor, streaming: bool, chunk_size: int = 50) -> Tensor:
    """The DiT's boolean attention mask (dit.py:163-166 -> mask.py:161-236).

    ``mask`` is the float padding mask ``[B,1,T]``; returns ``[B,1,T,T]``
    (True = visible).  Rows that would be all-False are forced True
    (mask.py:232-234).
    """
    pad = mask.bool()  # [B,1,T]
    T = pad.shape[-1]
    if streaming:
        masks = pad & subsequent_chunk_mask(T, chunk_size).unsqueeze(0)
    else:
        masks = pad.repeat(1, T, 1)
    empty = masks.sum(dim=-1) == 0
    if empty.any():
        masks = masks.clone()
        masks[empty] = True
    return masks.unsqueeze(1)


# --------------------------------------------------------------------------
# input embedding


def causal_conv_position_embedding(sd: StateDict, h: Tensor, kernel_size: int = 31,
                                   groups: int = 16) -> Tensor:
    """``CausalConvPositionEmbedding.forward`` with ``mask=None`` (modules.py:129-144).

    ``h`` is ``[B,T,C]``; left zero-pad by ``kernel_size-1`` before each grouped conv.
    """
    pre = "input_embed.conv_pos_embed."
    y = h.permute(0, 2, 1)
    y = F.pad(y, (kernel_size - 1, 0))
    y = mish(F.conv1d(y, sd[pre + "conv1.0.weight"], sd[pre + "conv1.0.bias"], groups=groups))
    y = F.pad(y, (kernel_size - 1, 0))
    y = mish(F.conv1d(y, sd[pre + "conv2.0.weight"], sd[pre + "conv2.0.bias"], groups=groups))
    return y.permute(0, 2, 1)


def input_embedding(sd: StateDict, x: Tensor, cond: Tensor, mu: Tensor, spks: Tensor) -> Tensor:
    """``InputEmbedding.forward`` (dit.py:84-98).  All inputs frame-major ``[B,T,80]``; spks ``[B,80]``."""
    spk = spks[:, None, :].expand(-1, x.shape[1], -1)
    h = F.linear(torch.cat([x, cond, mu, spk], dim=-1),
                 sd["input_embed.proj.weight"], sd["input_embed.proj.bias"])
    return causal_conv_position_embedding(sd, h) + h


# --------------------------------------------------------------------------
# transformer block


def block_modulation(sd: StateDict, index: int, temb: Tensor) -> tuple[Tensor, ...]:
    """``AdaLayerNormZero`` projection (modules.py:239-241): 6 chunks in the order
    shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp."""
    pre = f"transformer_blocks.{index}.attn_norm.linear."
    emb = F.linear(F.silu(temb), sd[pre + "weight"], sd[pre + "bias"])
    return torch.chunk(emb, 6, dim=1)


def final_modulation(sd: StateDict, temb: Tensor) -> tuple[Tensor, Tensor]:
    """``AdaLayerNormZero_Final`` projection (modules.py:260-262): (scale, shift) order."""
    emb = F.linear(F.silu(temb), sd["norm_out.linear.weight"], sd["norm_out.linear.bias"])
    scale, shift = torch.chunk(emb, 2, dim=1)
    return scale, shift


def attention(sd: StateDict, index: int, x: Tensor, attn_mask: Tensor | None, freqs: Tensor | None,
              heads: int) -> Tensor:
    """``Attention`` + ``AttnProcessor.__call__`` (modules.py:353-407)."""
    pre = f"transformer_blocks.{index}.attn."
    batch = x.shape[0]
    q = F.linear(x, sd[pre + "to_q.weight"], sd[pre + "to_q.bias"])
    k = F.linear(x, sd[pre + "to_k.weight"], sd[pre + "to_k.bias"])
    v = F.linear(x, sd[pre + "to_v.weight"], sd[pre + "to_v.bias"])
    if freqs is not None:
        q = apply_rotary(q, freqs)
        k = apply_rotary(k, freqs)
    head_dim = k.shape[-1] // heads
    q = q.view(batch, -1, heads, head_dim).transpose(1, 2)
    k = k.view(batch, -1, heads, head_dim).transpose(1, 2)
    v = v.view(batch, -1, heads, head_dim).transpose(1, 2)
    o = F.scaled_dot_product_attention(q, k, v, attn_mask=attn_mask, dropout_p=0.0, is_causal=False)
    o = o.transpose(1, 2).reshape(batch, -1, heads * head_dim)
    o = F.linear(o, sd[pre + "to_out.0.weight"], sd[pre + "to_out.0.bias"])
    if attn_mask is not None:
        # modules.py:400-405: zero the output where the last mask row hides the key.
        keep = attn_mask[:, 0, -1].unsqueeze(-1)
        o = o.masked_fill(~keep, 0.0)
    return o


def feed_forward(sd: StateDict, index: int, x: Tensor) -> Tensor:
    """``FeedForward`` (modules.py:271-282): Linear -> tanh-GELU -> (Dropout, eval no-op) -> Linear."""
    pre = f"transformer_blocks.{index}.ff.ff."
    hidden = gelu_tanh(F.linear(x, sd[pre + "0.0.weight"], sd[pre + "0.0.bias"]))
    return F.linear(hidden, sd[pre + "2.weight"], sd[pre + "2.bias"])


def dit_block(sd: StateDict, index: int, x: Tensor, temb: Tensor, attn_mask: Tensor | None,
              freqs: Tensor | None, heads: int) -> Tensor:
    """``DiTBlock.forward`` (modules.py:516-530)."""
    shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = block_modulation(sd, index, temb)
    norm = layer_norm(x) * (1 + scale_msa[:, None]) + shift_msa[:, None]
    attn_out = attention(sd, index, norm, attn_mask, freqs, heads)
    x = x + gate_msa.unsqueeze(1) * attn_out
    ff_norm = layer_norm(x) * (1 + scale_mlp[:, None]) + shift_mlp[:, None]
    x = x + gate_mlp.unsqueeze(1) * feed_forward(sd, index, ff_norm)
    return x


# --------------------------------------------------------------------------
# whole estimator


def infer_dims(sd: StateDict) -> dict:
    """Read (dim, depth) from a state dict laid out like the reference DiT."""
    dim = sd["proj_out.weight"].shape[1]
    depth = 0
    while f"transformer_blocks.{depth}.attn.to_q.weight" in sd:
        depth += 1
    return {"dim": dim, "depth": depth}


@torch.no_grad()
def dit_forward(sd: StateDict, x: Tensor, mask: Tensor, mu: Tensor, t: Tensor, spks: Tensor,
                cond: Tensor, streaming: bool = False, heads: int = 16, dim_head: int = 64,
                chunk_size: int = 50) -> Tensor:
    """``DiT.forward`` (dit.py:145-176), padded layout.

    x, mu, cond: ``[B,80,T]``; mask ``[B,1,T]``; t ``[B]`` (or scalar); spks ``[B,80]``.
    Returns ``[B,80,T]``.
    """
    depth = infer_dims(sd)["depth"]
    x = x.float().transpose(1, 2)
    mu = mu.float().transpose(1, 2)
    cond = cond.float().transpose(1, 2)
    spks = spks.float()
    batch, seq_len = x.shape[0], x.shape[1]
    t = t.float()
    if t.ndim == 0:
        t = t.repeat(batch)
    temb = timestep_embedding(sd, t)
    h = input_embedding(sd, x, cond, mu, spks)
    freqs = rotary_freqs(torch.arange(seq_len), dim_head)
    attn_mask = attention_mask(mask, streaming, chunk_size)
    for index in range(depth):
        h = dit_block(sd, index, h, temb, attn_mask, freqs, heads)
    scale, shift = final_modulation(sd, temb)
    h = layer_norm(h) * (1 + scale)[:, None, :] + shift[:, None, :]
    out = F.linear(h, sd["proj_out.weight"], sd["proj_out.bias"])
    return out.transpose(1, 2)


# --------------------------------------------------------------------------
# solver


def cosine_schedule(n_steps: int) -> Tensor:
    """``1 - cos(linspace(0,1,n+1) * pi/2)`` (flashinfer_flow.py:34-41; flow_matching.py:66-68)."""
    span = torch.linspace(0, 1, n_steps + 1, dtype=torch.float32)
    return 1 - torch.cos(span * 0.5 * torch.pi)


@torch.no_grad()
def solve_euler_batched(estimator: Callable[..., Tensor], noise: Tensor, mu: Tensor, mask: Tensor,
                        spks: Tensor, cond: Tensor, n_steps: int = 10, cfg_rate: float = 0.7,
                        streaming: bool = False, on_step: Callable | None = None) -> Tensor:
    """``solve_euler_batched`` (flashinfer_flow.py:16-74): 2B CFG stack
    ``[cond_0..cond_{B-1}, uncond_0..uncond_{B-1}]`` with zeroed mu/spks/cond in the
    unconditional half, then ``x += dt * ((1+cfg) v_c - cfg v_u)``.

    ``estimator(x, mask, mu, t, spks, cond, streaming)`` returns ``[2B,80,T]``.
    ``on_step(step, velocity, sample)`` is an optional observer for per-step checks.
    """
    batch = mu.shape[0]
    span = cosine_schedule(n_steps)
    time = span[0]
    step_size = span[1] - span[0]
    mask_in = mask.repeat(2, 1, 1).float()
    mu_in = torch.cat([mu, torch.zeros_like(mu)], dim=0).float()
    spk_in = torch.cat([spks, torch.zeros_like(spks)], dim=0).float()
    cond_in = torch.cat([cond, torch.zeros_like(cond)], dim=0).float()
    t_in = torch.zeros(2 * batch)
    sample = noise.float()
    for step in range(1, len(span)):
        t_in.fill_(float(time))
        velocity = estimator(sample.repeat(2, 1, 1), mask_in, mu_in, t_in, spk_in, cond_in, streaming)
        conditional, unconditional = torch.split(velocity, [batch, batch], dim=0)
        derivative = (1.0 + cfg_rate) * conditional - cfg_rate * unconditional
        if on_step is not None:
            on_step(step, velocity, sample)
        sample = sample + step_size * derivative
        time = time + step_size
        if step < len(span) - 1:
            step_size = span[step + 1] - time
    return sample


# --------------------------------------------------------------------------
# packed <-> padded helpers (flashinfer_dit.py:364-405,535-543)


def lengths_from_mask(mask: Tensor) -> list[int]:
    """Document lengths as the reference takes them: ``mask[:,0].sum(-1)`` (flashinfer_dit.py:460)."""
    return [int(v) for v in mask[:, 0].sum(-1).round().long().tolist()]


def cu_seqlens(lengths: Sequence[int]) -> list[int]:
    """Exclusive prefix sum (flashinfer_attention.py:82-86)."""
    out = [0]
    for n in lengths:
        out.append(out[-1] + int(n))
    return out


def pack(padded: Tensor, lengths: Sequence[int]) -> Tensor:
    """``[B,C,T]`` -> packed rows ``[R,C]`` (doc-major, frame order kept)."""
    return torch.cat([padded[b, :, :n].transpose(0, 1) for b, n in enumerate(lengths)], dim=0)


def unpack(rows: Tensor, lengths: Sequence[int], padded_len: int) -> Tensor:
    """Packed rows ``[R,C]`` -> ``[B,C,T]`` with zeros in padded frames (flashinfer_dit.py:536-543)."""
    out = rows.new_zeros(len(lengths), rows.shape[1], padded_len)
    offset = 0
    for b, n in enumerate(lengths):
        out[b, :, :n] = rows[offset:offset + n].transpose(0, 1)
        offset += n
    return out


@torch.no_grad()
def dit_forward_packed(sd: StateDict, x: Tensor, mu: Tensor, cond: Tensor, spks: Tensor, t: Tensor,
                       seqlens: Sequence[int], streaming: bool = False, heads: int = 16,
                       chunk_size: int = 50) -> Tensor:
    """Packed-row view of ``dit_forward``: each document runs unpadded on its own.

    x, mu, cond: ``[R,80]``; spks ``[N,80]``; t ``[N]`` or ``[1]``.  Returns ``[R,80]``.
    Documents are independent in the reference (mask.py + causal conv), so
    this equals ``dit_forward`` on the padded batch restricted to valid frames.
    """
    outs = []
    cu = cu_seqlens(seqlens)
    for d, n in enumerate(seqlens):
        rows = slice(cu[d], cu[d + 1])
        td = t[d if t.numel() > 1 else 0].reshape(1)
        outs.append(dit_forward(
            sd, x[rows].T[None], torch.ones(1, 1, n), mu[rows].T[None], td, spks[d:d + 1],
            cond[rows].T[None], streaming=streaming, heads=heads, chunk_size=chunk_size,
        )[0].T)
    return torch.cat(outs, dim=0)
