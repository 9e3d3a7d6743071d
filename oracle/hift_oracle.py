"""fp32/fp64 CPU restatement of the CosyVoice3 HiFT vocoder (``CausalHiFTGenerator.inference``).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Paths are relative to
``faster_cosyvoice/token2wav/cosyvoice/``.

* weight norm folded as ``v * (g / ||v||)`` over all but the output dim
  (torch ``weight_norm`` parametrization, used by generator.py:26-29);
* ``CausalConv1d`` / ``CausalConv1dDownSample`` / ``CausalConv1dUpsample``
  (transformer/convolution.py:150-263): left or right zero padding (or a context "cache"),
  stride with ``stride - 1`` left padding, nearest upsampling then ``k - 1`` left padding;
* ``Snake`` x + sin(a x)^2 / (a + 1e-9) (transformer/activation.py:73-84); ``ResBlock``
  (generator.py:46-116);
* ``CausalConvRNNF0Predictor`` in fp64 (hifigan/f0_predictor.py:62-103);
* ``SineGen2`` / ``SourceModuleHnNSF`` in causal inference mode with their fixed random buffers
  (generator.py:192-381);
* ``CausalHiFTGenerator.decode`` / ``inference`` (generator.py:497-511, 674-735): STFT of the
  source, conv_pre, three upsampling stages each fused with the down-sampled source, mean of the
  resblocks, conv_post, exp/sin, iSTFT, clamp; ``finalize=False`` keeps the right context.
"""

from __future__ import annotations

from typing import Mapping

import numpy as np
import torch
import torch.nn.functional as F

Tensor = torch.Tensor

_G = ".parametrizations.weight.original0"
_V = ".parametrizations.weight.original1"


def fold_weight_norm(sd: Mapping[str, Tensor]) -> dict[str, Tensor]:
    """Replace every (g, v) parametrization pair by the effective ``weight``.  The F0
    predictor's parameters are folded and kept in fp64, as the reference casts that module to
    fp64 before use (generator.py:722), so its parametrization runs in fp64."""
    out = {}
    for k, v in sd.items():
        f0 = k.startswith("f0_predictor.")
        if k.endswith(_G):
            name = k[: -len(_G)]
            g, vv = v, sd[name + _V]
            if f0:
                g, vv = g.double(), vv.double()
            norm = vv.flatten(1).norm(dim=1).view(-1, *([1] * (vv.dim() - 1)))
            out[name + ".weight"] = vv * (g / norm)
        elif not k.endswith(_V):
            out[k] = v.double() if f0 else v
    return out


def causal_padding(k: int, dilation: int = 1) -> int:
    """convolution.py:172."""
    return int((k * dilation - dilation) / 2) * 2 + (k + 1) % 2


def causal_conv(x: Tensor, w: Tensor, b: Tensor, dilation: int = 1, right: bool = False,
                cache: Tensor | None = None) -> Tensor:
    """``CausalConv1d``: zero (or ``cache``) padding on the left, or on the right for the
    lookahead type; output length = input length."""
    pad = causal_padding(w.shape[2], dilation)
    if cache is None:
        cache = x.new_zeros(x.shape[0], x.shape[1], pad)
    assert cache.shape[2] == pad
    x = torch.cat([x, cache], dim=2) if right else torch.cat([cache, x], dim=2)
    return F.conv1d(x, w, b, dilation=dilation)


def down_conv(x: Tensor, w: Tensor, b: Tensor, stride: int) -> Tensor:
    """``CausalConv1dDownSample``: ``stride - 1`` zeros on the left, then a strided conv."""
    return F.conv1d(F.pad(x, (stride - 1, 0)), w, b, stride=stride)


def up_conv(x: Tensor, w: Tensor, b: Tensor, rate: int) -> Tensor:
    """``CausalConv1dUpsample``: nearest upsampling by ``rate``, ``k - 1`` zeros on the left."""
    x = F.interpolate(x, scale_factor=rate, mode="nearest")
    return F.conv1d(F.pad(x, (w.shape[2] - 1, 0)), w, b)


def snake(x: Tensor, alpha: Tensor) -> Tensor:
    a = alpha.view(1, -1, 1)
    return x + (1.0 / (a + 1e-9)) * torch.pow(torch.sin(x * a), 2)


def resblock(sd: Mapping[str, Tensor], name: str, x: Tensor, dilations) -> Tensor:
    for j, d in enumerate(dilations):
        t = snake(x, sd[f"{name}.activations1.{j}.alpha"])
        t = causal_conv(t, sd[f"{name}.convs1.{j}.weight"], sd[f"{name}.convs1.{j}.bias"], d)
        t = snake(t, sd[f"{name}.activations2.{j}.alpha"])
        t = causal_conv(t, sd[f"{name}.convs2.{j}.weight"], sd[f"{name}.convs2.{j}.bias"], 1)
        x = t + x
    return x


def f0_predict(sd: Mapping[str, Tensor], mel: Tensor, finalize: bool = True) -> Tensor:
    """F0 in fp64 from Mel ``[B, 80, T]``: ``[B, T]`` (``[B, T - 3]`` when not finalizing: the
    first conv's 3-frame lookahead becomes right context)."""
    g = lambda k: sd[f"f0_predictor.{k}"].double()
    x = mel.double()
    w0, b0 = g("condnet.0.weight"), g("condnet.0.bias")
    if finalize:
        x = causal_conv(x, w0, b0, right=True)
    else:
        pad = causal_padding(w0.shape[2])
        x = causal_conv(x[:, :, :-pad], w0, b0, right=True, cache=x[:, :, -pad:])
    x = F.elu(x)
    for i in (2, 4, 6, 8):
        x = F.elu(causal_conv(x, g(f"condnet.{i}.weight"), g(f"condnet.{i}.bias")))
    y = F.linear(x.transpose(1, 2), g("classifier.weight"), g("classifier.bias"))
    return torch.abs(y.squeeze(-1))


def source(sd: Mapping[str, Tensor], f0: Tensor, buffers: Mapping[str, Tensor], dims) -> Tensor:
    """Harmonic source ``[B, 1, L]`` from frame F0 ``[B, T]`` (fp32), L = T * upsample_scale:
    nearest-upsampled F0, per-harmonic phase accumulated at frame rate and held over each frame,
    voiced sines plus table noise, merged by a Linear + tanh."""
    scale = dims.upsample_scale
    H = dims.nb_harmonics + 1
    f0_up = F.interpolate(f0[:, None], scale_factor=scale, mode="nearest").transpose(1, 2)
    fn = f0_up * torch.arange(1, H + 1, dtype=torch.float32).view(1, 1, -1)
    rad = (fn / dims.sampling_rate) % 1
    rad[:, 0, :] = rad[:, 0, :] + buffers["rand_ini"]
    rad = F.interpolate(rad.transpose(1, 2), scale_factor=1 / scale, mode="linear").transpose(1, 2)
    phase = torch.cumsum(rad, dim=1) * 2 * np.pi
    phase = F.interpolate(phase.transpose(1, 2) * scale, scale_factor=scale,
                          mode="nearest").transpose(1, 2)
    sines = torch.sin(phase) * dims.nsf_alpha
    uv = (f0_up > dims.nsf_voiced_threshold).type(torch.float32)
    noise_amp = uv * dims.nsf_sigma + (1 - uv) * dims.nsf_alpha / 3
    noise = noise_amp * buffers["sine_waves"][:, :sines.shape[1]]
    waves = sines * uv + noise
    merged = torch.tanh(F.linear(waves, sd["m_source.l_linear.weight"], sd["m_source.l_linear.bias"]))
    return merged.transpose(1, 2)


def _window(n_fft: int) -> Tensor:
    """Periodic Hann window (scipy get_window("hann", n, fftbins=True))."""
    k = torch.arange(n_fft, dtype=torch.float64)
    return (0.5 - 0.5 * torch.cos(2 * np.pi * k / n_fft)).float()


def stft(x: Tensor, dims) -> tuple[Tensor, Tensor]:
    spec = torch.stft(x, dims.n_fft, dims.hop_len, dims.n_fft, window=_window(dims.n_fft),
                      return_complex=True)
    spec = torch.view_as_real(spec)
    return spec[..., 0], spec[..., 1]


def istft(magnitude: Tensor, phase: Tensor, dims) -> Tensor:
    magnitude = torch.clip(magnitude, max=1e2)
    spec = torch.complex(magnitude * torch.cos(phase), magnitude * torch.sin(phase))
    return torch.istft(spec, dims.n_fft, dims.hop_len, dims.n_fft, window=_window(dims.n_fft))


def decode(sd: Mapping[str, Tensor], x: Tensor, s: Tensor, dims, finalize: bool = True) -> Tensor:
    re, im = stft(s.squeeze(1), dims)
    look = dims.conv_pre_look_right
    if finalize:
        x = causal_conv(x, sd["conv_pre.weight"], sd["conv_pre.bias"], right=True)
    else:
        x = causal_conv(x[:, :, :-look], sd["conv_pre.weight"], sd["conv_pre.bias"], right=True,
                        cache=x[:, :, -look:])
        cut = int(np.prod(dims.upsample_rates)) * look
        re, im = re[:, :, :-cut], im[:, :, :-cut]
    s_stft = torch.cat([re, im], dim=1)
    n_stage = len(dims.upsample_rates)
    n_res = len(dims.resblock_kernel_sizes)
    for i, rate in enumerate(dims.upsample_rates):
        x = F.leaky_relu(x, dims.lrelu_slope)
        x = up_conv(x, sd[f"ups.{i}.weight"], sd[f"ups.{i}.bias"], rate)
        if i == n_stage - 1:
            x = F.pad(x, (1, 0), mode="reflect")
        k, stride = dims.source_down(i)
        w, b = sd[f"source_downs.{i}.weight"], sd[f"source_downs.{i}.bias"]
        si = causal_conv(s_stft, w, b) if stride == 1 else down_conv(s_stft, w, b, stride)
        si = resblock(sd, f"source_resblocks.{i}", si, dims.source_resblock_dilation_sizes[i])
        x = x + si
        xs = None
        for j in range(n_res):
            r = resblock(sd, f"resblocks.{i * n_res + j}", x, dims.resblock_dilation_sizes[j])
            xs = r if xs is None else xs + r
        x = xs / n_res
    x = F.leaky_relu(x)
    x = causal_conv(x, sd["conv_post.weight"], sd["conv_post.bias"])
    half = dims.n_fft // 2 + 1
    y = istft(torch.exp(x[:, :half, :]), torch.sin(x[:, half:, :]), dims)
    if not finalize:
        y = y[:, :-int(np.prod(dims.upsample_rates) * dims.hop_len)]
    return torch.clamp(y, -dims.audio_limit, dims.audio_limit)


@torch.no_grad()
def inference(sd: Mapping[str, Tensor], mel: Tensor, buffers: Mapping[str, Tensor], dims,
              finalize: bool = True) -> tuple[Tensor, Tensor]:
    """``CausalHiFTGenerator.inference``: (waveform ``[B, N]``, source ``[B, 1, L]``).
    ``sd``: the state dict with weight norm folded (``fold_weight_norm``)."""
    f0 = f0_predict(sd, mel, finalize).to(mel.dtype)
    s = source(sd, f0, buffers, dims)
    if finalize:
        speech = decode(sd, mel, s, dims, True)
    else:
        pad = causal_padding(sd["f0_predictor.condnet.0.weight"].shape[2])
        speech = decode(sd, mel[:, :, :-pad], s, dims, False)
    return speech, s
