"""Seeded synthetic weights and packed workloads for the DiT estimator path.

Real ``flow.pt`` weights are not available offline, so every measurement and
parity test runs on seeded random-init weights with the reference DiT's
state-dict layout (``cosyvoice/flow/DiT/dit.py:104-143``, hyper-parameters from
``builders.py:17-21``) and on seeded synthetic inputs.

Draws use numpy's PCG64 ``Generator`` (float32 normal draws),
which is platform independent, so the same seed gives the same tensors on any
host.  Defaults: weights from seed 0, tensors from seed 1234, layouts from
seed 0.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

MEL = 80
TEMB_FREQ = 256


@dataclass(frozen=True)
class DiTDims:
    """Shape of the CosyVoice3 DiT (builders.py:17-21)."""

    dim: int = 1024
    depth: int = 22
    heads: int = 16
    dim_head: int = 64
    ff_mult: int = 2
    mel_dim: int = MEL
    conv_kernel: int = 31
    conv_groups: int = 16

    @property
    def ff_dim(self) -> int:
        return self.dim * self.ff_mult

    @property
    def in_dim(self) -> int:
        return 4 * self.mel_dim  # x, cond, mu, spks (dit.py:91-96)


def state_dict_shapes(d: DiTDims) -> list[tuple[str, tuple[int, ...]]]:
    """Parameter names and shapes in the reference's registration order."""
    out: list[tuple[str, tuple[int, ...]]] = [
        ("time_embed.time_mlp.0.weight", (d.dim, TEMB_FREQ)),
        ("time_embed.time_mlp.0.bias", (d.dim,)),
        ("time_embed.time_mlp.2.weight", (d.dim, d.dim)),
        ("time_embed.time_mlp.2.bias", (d.dim,)),
        ("input_embed.proj.weight", (d.dim, d.in_dim)),
        ("input_embed.proj.bias", (d.dim,)),
    ]
    cpg = d.dim // d.conv_groups
    for conv in ("conv1", "conv2"):
        out.append((f"input_embed.conv_pos_embed.{conv}.0.weight", (d.dim, cpg, d.conv_kernel)))
        out.append((f"input_embed.conv_pos_embed.{conv}.0.bias", (d.dim,)))
    inner = d.heads * d.dim_head
    for i in range(d.depth):
        p = f"transformer_blocks.{i}."
        out += [
            (p + "attn_norm.linear.weight", (6 * d.dim, d.dim)),
            (p + "attn_norm.linear.bias", (6 * d.dim,)),
            (p + "attn.to_q.weight", (inner, d.dim)),
            (p + "attn.to_q.bias", (inner,)),
            (p + "attn.to_k.weight", (inner, d.dim)),
            (p + "attn.to_k.bias", (inner,)),
            (p + "attn.to_v.weight", (inner, d.dim)),
            (p + "attn.to_v.bias", (inner,)),
            (p + "attn.to_out.0.weight", (d.dim, inner)),
            (p + "attn.to_out.0.bias", (d.dim,)),
            (p + "ff.ff.0.0.weight", (d.ff_dim, d.dim)),
            (p + "ff.ff.0.0.bias", (d.ff_dim,)),
            (p + "ff.ff.2.weight", (d.dim, d.ff_dim)),
            (p + "ff.ff.2.bias", (d.dim,)),
        ]
    out += [
        ("norm_out.linear.weight", (2 * d.dim, d.dim)),
        ("norm_out.linear.bias", (2 * d.dim,)),
        ("proj_out.weight", (d.mel_dim, d.dim)),
        ("proj_out.bias", (d.mel_dim,)),
    ]
    return out


def random_state_dict(dims: DiTDims = DiTDims(), seed: int = 0, std: float = 0.02,
                      gate_bias: float = 0.0, qk_std: float | None = None
                      ) -> dict[str, torch.Tensor]:
    """Every parameter ~ N(0, std), drawn in registration order from one PCG64 stream.

    ``gate_bias`` (>0) adds a constant to the AdaLN gate biases (chunks 2 and 5
    of each block's 6-way modulation) so that every block changes the
    residual stream by O(gate_bias); the default keeps plain N(0, 0.02),
    where the gates are small but nonzero.

    ``qk_std`` (when given) draws the ``to_q`` / ``to_k`` weights with that deviation instead
    (the same draws, rescaled).  With unit-variance normalised inputs the attention logits
    q.k/8 then have a deviation of about ``1024 qk_std^2`` (0.4 at 0.02, 3.7 at 0.06), so the
    softmax is peaked and the output depends on which keys are visible and on RoPE.
    """
    rng = np.random.Generator(np.random.PCG64(seed))
    sd = {}
    for name, shape in state_dict_shapes(dims):
        sigma = std
        if qk_std is not None and (name.endswith("to_q.weight") or name.endswith("to_k.weight")):
            sigma = qk_std
        arr = rng.standard_normal(int(np.prod(shape)), dtype=np.float32) * np.float32(sigma)
        sd[name] = torch.from_numpy(arr.reshape(shape))
    if gate_bias:
        for i in range(dims.depth):
            b = sd[f"transformer_blocks.{i}.attn_norm.linear.bias"].view(6, dims.dim)
            b[2] += gate_bias
            b[5] += gate_bias
    return sd


# --------------------------------------------------------------------------
# Flow front-end (token embedding, PreLookaheadLayer, speaker projection)


@dataclass(frozen=True)
class FlowDims:
    """Front-end shapes of ``CausalMaskedDiffWithDiT`` (builders.py:29-35)."""

    vocab: int = 6561
    feat: int = MEL
    channels: int = 1024
    lookahead: int = 3
    spk_dim: int = 192
    token_mel_ratio: int = 2


def flow_state_dict_shapes(d: FlowDims = FlowDims()) -> list[tuple[str, tuple[int, ...]]]:
    """Front-end parameter names and shapes as they sit in a flow state dict
    (flow.py:307-310, upsample_encoder.py:61-70)."""
    return [
        ("input_embedding.weight", (d.vocab, d.feat)),
        ("spk_embed_affine_layer.weight", (d.feat, d.spk_dim)),
        ("spk_embed_affine_layer.bias", (d.feat,)),
        ("pre_lookahead_layer.conv1.weight", (d.channels, d.feat, d.lookahead + 1)),
        ("pre_lookahead_layer.conv1.bias", (d.channels,)),
        ("pre_lookahead_layer.conv2.weight", (d.feat, d.channels, 3)),
        ("pre_lookahead_layer.conv2.bias", (d.feat,)),
    ]


def random_flow_state_dict(dims: FlowDims = FlowDims(), seed: int = 0) -> dict[str, torch.Tensor]:
    """Embedding rows ~ N(0, 1) (nn.Embedding's init); every other parameter ~ N(0, 1/fan_in),
    fan_in = input width of the layer the parameter belongs to, so activations stay O(1).
    Drawn in ``flow_state_dict_shapes`` order from one PCG64 stream."""
    fan_in = {"input_embedding": 1, "spk_embed_affine_layer": dims.spk_dim,
              "pre_lookahead_layer.conv1": dims.feat * (dims.lookahead + 1),
              "pre_lookahead_layer.conv2": dims.channels * 3}
    rng = np.random.Generator(np.random.PCG64(seed))
    sd = {}
    for name, shape in flow_state_dict_shapes(dims):
        std = np.float32(1.0 / np.sqrt(fan_in[name.rsplit(".", 1)[0]]))
        arr = rng.standard_normal(int(np.prod(shape)), dtype=np.float32) * std
        sd[name] = torch.from_numpy(arr.reshape(shape))
    return sd


# --------------------------------------------------------------------------
# HiFT vocoder (CausalHiFTGenerator + CausalConvRNNF0Predictor)


@dataclass(frozen=True)
class HiFTDims:
    """Shape of the CosyVoice3 HiFT vocoder (builders.py:38-50)."""

    in_channels: int = MEL
    base_channels: int = 512
    nb_harmonics: int = 8
    sampling_rate: int = 24000
    nsf_alpha: float = 0.1
    nsf_sigma: float = 0.003
    nsf_voiced_threshold: float = 10.0
    upsample_rates: tuple = (8, 5, 3)
    upsample_kernel_sizes: tuple = (16, 11, 7)
    n_fft: int = 16
    hop_len: int = 4
    resblock_kernel_sizes: tuple = (3, 7, 11)
    resblock_dilation_sizes: tuple = ((1, 3, 5), (1, 3, 5), (1, 3, 5))
    source_resblock_kernel_sizes: tuple = (7, 7, 11)
    source_resblock_dilation_sizes: tuple = ((1, 3, 5), (1, 3, 5), (1, 3, 5))
    lrelu_slope: float = 0.1
    audio_limit: float = 0.99
    conv_pre_look_right: int = 4
    f0_channels: int = 512

    @property
    def upsample_scale(self) -> int:
        """Waveform samples per Mel frame (prod(upsample_rates) * hop_len)."""
        out = self.hop_len
        for r in self.upsample_rates:
            out *= r
        return out

    def stage_channels(self, i: int) -> int:
        return self.base_channels // (2 ** (i + 1))

    def source_down(self, i: int) -> tuple[int, int]:
        """(kernel, stride) of source_downs[i]: the STFT frames of the source, brought to the
        rate of upsampling stage i (generator.py:640-655)."""
        rates = [1] + list(self.upsample_rates[::-1][:-1])
        cum = list(np.cumprod(rates))[::-1]
        u = int(cum[i])
        return (1, 1) if u == 1 else (2 * u, u)


def _wn(name: str, shape: tuple[int, ...]) -> list[tuple[str, tuple[int, ...]]]:
    """A weight-normalised conv: parametrizations g [out,1,1], v [out,in,k], then bias."""
    return [(f"{name}.parametrizations.weight.original0", (shape[0], 1, 1)),
            (f"{name}.parametrizations.weight.original1", shape),
            (f"{name}.bias", (shape[0],))]


def _resblock_shapes(name: str, ch: int, k: int, dils) -> list[tuple[str, tuple[int, ...]]]:
    out = []
    for j in range(len(dils)):
        out += _wn(f"{name}.convs1.{j}", (ch, ch, k))
    for j in range(len(dils)):
        out += _wn(f"{name}.convs2.{j}", (ch, ch, k))
    out += [(f"{name}.activations1.{j}.alpha", (ch,)) for j in range(len(dils))]
    out += [(f"{name}.activations2.{j}.alpha", (ch,)) for j in range(len(dils))]
    return out


def hift_state_dict_shapes(d: HiFTDims = HiFTDims()) -> list[tuple[str, tuple[int, ...]]]:
    """Parameter names and shapes of ``CausalHiFTGenerator`` in registration order
    (generator.py:578-675, f0_predictor.py:59-90), as ``hift.pt`` stores them once the
    ``generator.`` prefix is removed (token2wav.py:71-74)."""
    H = d.nb_harmonics + 1
    spec = d.n_fft + 2
    out = [("m_source.l_linear.weight", (1, H)), ("m_source.l_linear.bias", (1,))]
    out += _wn("conv_pre", (d.base_channels, d.in_channels, d.conv_pre_look_right + 1))
    for i, k in enumerate(d.upsample_kernel_sizes):
        out += _wn(f"ups.{i}", (d.stage_channels(i), d.base_channels // (2 ** i), k))
    for i in range(len(d.upsample_rates)):
        k, _ = d.source_down(i)
        out += [(f"source_downs.{i}.weight", (d.stage_channels(i), spec, k)),
                (f"source_downs.{i}.bias", (d.stage_channels(i),))]
    for i, (k, dil) in enumerate(zip(d.source_resblock_kernel_sizes,
                                     d.source_resblock_dilation_sizes)):
        out += _resblock_shapes(f"source_resblocks.{i}", d.stage_channels(i), k, dil)
    n = 0
    for i in range(len(d.upsample_rates)):
        for k, dil in zip(d.resblock_kernel_sizes, d.resblock_dilation_sizes):
            out += _resblock_shapes(f"resblocks.{n}", d.stage_channels(i), k, dil)
            n += 1
    out += _wn("conv_post", (spec, d.stage_channels(len(d.upsample_rates) - 1), 7))
    C = d.f0_channels
    out += _wn("f0_predictor.condnet.0", (C, d.in_channels, 4))
    for i in (2, 4, 6, 8):
        out += _wn(f"f0_predictor.condnet.{i}", (C, C, 3))
    out += [("f0_predictor.classifier.weight", (1, C)), ("f0_predictor.classifier.bias", (1,))]
    return out


def random_hift_state_dict(dims: HiFTDims = HiFTDims(), seed: int = 0,
                           post_gain: float = 0.3) -> dict[str, torch.Tensor]:
    """Seeded HiFT parameters with O(1) activations: weight-norm directions v ~ N(0, 1),
    gains g ~ N(1, 0.1) (so each conv keeps the variance of its input), biases and the source
    merge ~ N(0, 0.1), Snake alphas ~ U(0.5, 1.5); ``post_gain`` scales conv_post's gains so
    the log-magnitudes stay near 0 and the waveform is not clamped.  The F0 head gets weights
    ~ N(0, 2) and a bias of 10 Hz, so F0 = |10 + O(5)| Hz straddles the 10 Hz voicing threshold
    and both the voiced and the unvoiced source branches are exercised."""
    rng = np.random.Generator(np.random.PCG64(seed))
    sd = {}
    for name, shape in hift_state_dict_shapes(dims):
        n = int(np.prod(shape))
        if name.endswith("original0"):
            arr = 1.0 + 0.1 * rng.standard_normal(n, dtype=np.float32)
            if name.startswith("conv_post"):
                arr *= np.float32(post_gain)
        elif name.endswith("alpha"):
            arr = rng.uniform(0.5, 1.5, n).astype(np.float32)
        elif name.endswith("original1"):
            arr = rng.standard_normal(n, dtype=np.float32)
        elif name.startswith("source_downs") and name.endswith("weight"):
            arr = rng.standard_normal(n, dtype=np.float32) / np.float32(np.sqrt(n / shape[0]))
        else:
            arr = np.float32(0.1) * rng.standard_normal(n, dtype=np.float32)
        sd[name] = torch.from_numpy(arr.reshape(shape).astype(np.float32))
    sd["f0_predictor.classifier.weight"] = sd["f0_predictor.classifier.weight"] * 20.0
    sd["f0_predictor.classifier.bias"] = torch.full((1,), 10.0)
    return sd


def hift_macs_per_frame(d: HiFTDims = HiFTDims()) -> dict[str, int]:
    """Algorithmic multiply-adds of ``CausalHiFTGenerator.inference`` per Mel frame (real
    channel counts, no padding): fp32 convolutions by stage, and the fp64 F0 predictor."""
    spec = d.n_fft + 2
    out = {"conv_pre": d.in_channels * d.base_channels * (d.conv_pre_look_right + 1)}
    rows = 1
    cin = d.base_channels
    for i, (r, k) in enumerate(zip(d.upsample_rates, d.upsample_kernel_sizes)):
        rows *= r
        C = d.stage_channels(i)
        kd, _ = d.source_down(i)
        res = sum(len(dil) * 2 * C * C * kk for kk, dil in zip(d.resblock_kernel_sizes,
                                                               d.resblock_dilation_sizes))
        src = len(d.source_resblock_dilation_sizes[i]) * 2 * C * C * d.source_resblock_kernel_sizes[i]
        out[f"stage{i}"] = rows * (cin * C * k + spec * C * kd + res + src)
        cin = C
    out["conv_post"] = rows * cin * spec * 7
    out["f0_fp64"] = d.in_channels * d.f0_channels * 4 + 4 * d.f0_channels * d.f0_channels * 3
    return out


def random_hift_buffers(dims: HiFTDims = HiFTDims(), max_samples: int = 300 * 24000,
                        seed: int = 0) -> dict[str, torch.Tensor]:
    """The causal source's fixed random buffers (generator.py:223-226): initial harmonic
    phases ``rand_ini`` [1, H] with the fundamental's set to 0, and the uniform noise table
    ``sine_waves`` [1, max_samples, H].  The reference draws them from the global generator
    when the module is built; pass the reference's own buffers for sample-exact output."""
    g = torch.Generator().manual_seed(seed)
    H = dims.nb_harmonics + 1
    rand_ini = torch.rand(1, H, generator=g)
    rand_ini[:, 0] = 0
    return {"rand_ini": rand_ini, "sine_waves": torch.rand(1, max_samples, H, generator=g)}


# --------------------------------------------------------------------------
# packed workloads


@dataclass
class PackedBatch:
    """One packed CFG batch as the token2wav batcher hands it to the estimator.

    Rows are doc-major: documents ``0..B-1`` are the conditional halves,
    ``B..2B-1`` the unconditional halves (same lengths, zero mu/cond/spks),
    matching ``solve_euler_batched`` (flashinfer_flow.py:45-51).
    """

    name: str
    lengths: list[int]              # per request (B)
    prompt_lengths: list[int]       # prompt (cond) frames per request
    noise: torch.Tensor             # [Rc, 80] packed conditional rows
    mu: torch.Tensor                # [Rc, 80]
    cond: torch.Tensor              # [Rc, 80]
    spks: torch.Tensor              # [B, 80]
    streaming: bool = False
    n_steps: int = 10
    t: float | None = None          # fixed t for single-step configs
    meta: dict = field(default_factory=dict)

    @property
    def n_requests(self) -> int:
        return len(self.lengths)

    @property
    def doc_lengths(self) -> list[int]:
        """Packed document lengths including the CFG mirror (2B docs)."""
        return list(self.lengths) + list(self.lengths)

    @property
    def rows(self) -> int:
        return 2 * sum(self.lengths)

    def cfg_inputs(self) -> dict[str, torch.Tensor]:
        """Inputs for one estimator call over all 2B docs (x = noise in both halves)."""
        zeros = torch.zeros_like(self.mu)
        return {
            "x": torch.cat([self.noise, self.noise]),
            "mu": torch.cat([self.mu, zeros]),
            "cond": torch.cat([self.cond, zeros]),
            "spks": torch.cat([self.spks, torch.zeros_like(self.spks)]),
        }

    def padded(self) -> dict[str, torch.Tensor]:
        """Request-level padded tensors ``[B,80,T]`` as ``solve_euler_batched`` takes them."""
        T = max(self.lengths)
        B = self.n_requests
        out = {k: torch.zeros(B, MEL, T) for k in ("noise", "mu", "cond")}
        mask = torch.zeros(B, 1, T)
        off = 0
        for b, n in enumerate(self.lengths):
            for k in ("noise", "mu", "cond"):
                out[k][b, :, :n] = getattr(self, k)[off:off + n].T
            mask[b, 0, :n] = 1
            off += n
        out["mask"] = mask
        out["spks"] = self.spks.clone()
        return out


def _normal(rng: np.random.Generator, *shape: int) -> torch.Tensor:
    return torch.from_numpy(rng.standard_normal(int(np.prod(shape)), dtype=np.float32).reshape(shape))


def make_batch(name: str, lengths: list[int], prompt_lengths: list[int], seed: int = 1234,
               streaming: bool = False, n_steps: int = 10, t: float | None = None,
               meta: dict | None = None) -> PackedBatch:
    """Fill a batch layout with N(0,1) noise, mu and prompt mel (cond on the prompt frames only)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    rc = sum(lengths)
    noise = _normal(rng, rc, MEL)
    mu = _normal(rng, rc, MEL)
    prompt = _normal(rng, rc, MEL)
    spks = _normal(rng, len(lengths), MEL)
    cond = torch.zeros(rc, MEL)
    off = 0
    for n, p in zip(lengths, prompt_lengths):
        cond[off:off + p] = prompt[off:off + p]
        off += n
    return PackedBatch(name, list(lengths), list(prompt_lengths), noise, mu, cond, spks,
                       streaming=streaming, n_steps=n_steps, t=t, meta=meta or {})


def workload(index: int, layout_seed: int = 0, tensor_seed: int = 1234) -> PackedBatch:
    """The five benchmark workloads (numbered 1..5) of the estimator path.

    1. one block, 300 frames, full attention (CPU oracle case; use depth=1 weights);
    2. 22 layers, one request of 550 frames (prompt 250), CFG pair, one step;
    3. 8 requests, lengths U[100,1500], prompt fraction U(0.2,0.5), 10 steps;
    4. 32 streams, prefix U(150,400) + hop {30,60,120}, chunk-causal, 10 steps;
    5. 64 requests, lengths LogNormal(ln 800, 0.6) clipped to [64,3000], 10 steps.
    """
    rng = np.random.Generator(np.random.PCG64(layout_seed))
    if index == 1:
        t = float(rng.uniform(0.0, 1.0))
        b = make_batch("one_block_300", [300], [0], tensor_seed, n_steps=1, t=t)
        return b
    if index == 2:
        return make_batch("dit22_single_550", [550], [250], tensor_seed, n_steps=1, t=0.5)
    if index == 3:
        lengths = [int(v) for v in rng.integers(100, 1501, size=8)]
        fracs = rng.uniform(0.2, 0.5, size=8)
        prompts = [int(round(n * f)) for n, f in zip(lengths, fracs)]
        return make_batch("ragged8_cfg16_full", lengths, prompts, tensor_seed)
    if index == 4:
        prefix = [int(v) for v in rng.integers(150, 401, size=32)]
        hops = [int(v) for v in rng.choice([30, 60, 120], size=32)]
        lengths = [p + h for p, h in zip(prefix, hops)]
        return make_batch("stream32_cfg64_chunk50", lengths, prefix, tensor_seed, streaming=True,
                          meta={"hops": hops})
    if index == 5:
        raw = rng.lognormal(mean=math.log(800.0), sigma=0.6, size=64)
        lengths = [int(min(max(round(v), 64), 3000)) for v in raw]
        fracs = rng.uniform(0.2, 0.5, size=64)
        prompts = [int(round(n * f)) for n, f in zip(lengths, fracs)]
        return make_batch("lognormal64_cfg128_full", lengths, prompts, tensor_seed)
    raise ValueError(f"unknown workload {index}")


def flops_per_forward(doc_lengths: list[int], streaming: bool, dims: DiTDims = DiTDims(),
                      chunk: int = 50) -> dict[str, float]:
    """Algorithmic FLOPs of one DiT forward over packed docs.

    Dense per row: input proj 2*320*D, conv 2 * 2*31*(D/G)*D, per block
    2*D*(3D + D + 2F + F... ) i.e. QKV 6D^2, out 2D^2, FF 4DF, proj_out 2*D*80.
    Attention: 4*dim_head*heads FLOP per visible (q,k) pair per block.
    """
    D, F = dims.dim, dims.ff_dim
    per_row_dense = (2 * dims.in_dim * D
                     + 2 * (2 * dims.conv_kernel * (D // dims.conv_groups) * D)
                     + dims.depth * (2 * D * 3 * D + 2 * D * D + 2 * D * F + 2 * F * D)
                     + 2 * D * dims.mel_dim)
    rows = sum(doc_lengths)
    pairs = 0
    for n in doc_lengths:
        if streaming:
            q = np.arange(n)
            pairs += int(np.minimum((q // chunk + 1) * chunk, n).sum())
        else:
            pairs += n * n
    attn = 4.0 * dims.heads * dims.dim_head * pairs * dims.depth
    return {"dense": float(per_row_dense * rows), "attention": attn, "rows": rows,
            "pairs": pairs, "total": float(per_row_dense * rows) + attn}
