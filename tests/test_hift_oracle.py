"""CPU checks that pin the HiFT oracle (oracle/hift_oracle.py).

* ``hift_small.npz`` holds outputs of the reference's own ``CausalHiFTGenerator`` at reduced
  width (tests/golden/make_golden.py): F0, source and waveform, finalize True and False.  They
  pin the decode wiring, which no closed form fixes.
* Closed forms pin the pieces: weight-norm folding (row norms equal the gains), the causal
  padding rule, one-tap identity convolutions for the left, right (lookahead), strided and
  upsampling convolutions, Snake, the STFT/iSTFT pair (perfect reconstruction), and the sine
  source for a constant F0 with a zero noise table.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import hift_oracle as H

GOLDEN = Path(__file__).resolve().parent / "golden"


def _tuples(v):
    return tuple(_tuples(x) for x in v) if isinstance(v, list) else v


@pytest.fixture(scope="module")
def small(fcv):
    z = np.load(GOLDEN / "hift_small.npz")
    config = {k: _tuples(v) for k, v in json.loads(str(z["config"])).items()}
    dims = fcv.synthetic.HiFTDims(**config)
    sd = H.fold_weight_norm(fcv.synthetic.random_hift_state_dict(dims, seed=int(z["weight_seed"])))
    buf = {"rand_ini": torch.from_numpy(z["rand_ini"]), "sine_waves": torch.from_numpy(z["sine_waves"])}
    return z, dims, sd, buf


@pytest.mark.parametrize("finalize", [True, False])
def test_oracle_matches_reference_generator(small, finalize):
    z, dims, sd, buf = small
    tag = "fin" if finalize else "stream"
    mel = torch.from_numpy(z["mel"])
    f0 = H.f0_predict(sd, mel, finalize)
    torch.testing.assert_close(f0, torch.from_numpy(z[f"f0_{tag}"]), rtol=1e-12, atol=1e-12)
    speech, s = H.inference(sd, mel, buf, dims, finalize)
    torch.testing.assert_close(s, torch.from_numpy(z[f"s_{tag}"]), rtol=1e-6, atol=1e-6)
    ref = torch.from_numpy(z[f"speech_{tag}"])
    assert speech.shape == ref.shape
    torch.testing.assert_close(speech, ref, rtol=1e-5, atol=1e-5)
    # the fixture exercises both source branches and stays inside the clamp
    assert 0 < int((f0 > dims.nsf_voiced_threshold).sum()) < f0.numel()
    assert float(ref.abs().max()) < dims.audio_limit


def test_fold_weight_norm_row_norms_are_the_gains():
    g = torch.tensor([0.5, 2.0, 3.0]).view(3, 1, 1)
    v = torch.randn(3, 4, 5, generator=torch.Generator().manual_seed(0))
    sd = {"c.parametrizations.weight.original0": g, "c.parametrizations.weight.original1": v,
          "c.bias": torch.zeros(3)}
    w = H.fold_weight_norm(sd)["c.weight"]
    torch.testing.assert_close(w.flatten(1).norm(dim=1), g.flatten(), rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(w / w.flatten(1).norm(dim=1).view(3, 1, 1),
                               v / v.flatten(1).norm(dim=1).view(3, 1, 1), rtol=1e-6, atol=1e-6)


def test_causal_padding_rule():
    assert [H.causal_padding(k) for k in (1, 3, 4, 5, 7, 11)] == [0, 2, 3, 4, 6, 10]
    assert H.causal_padding(3, 5) == 10 and H.causal_padding(11, 3) == 30


def _tap(cout, cin, k, tap):
    w = torch.zeros(cout, cin, k)
    w[:, :, tap] = torch.eye(cout, cin)
    return w


def test_left_conv_tap_reads_back_by_dilation():
    """Left type: tap j of a dilation-d conv reads x[t - pad + j d] (zero before 0)."""
    x = torch.randn(1, 4, 20, generator=torch.Generator().manual_seed(1))
    k, d = 3, 3
    pad = H.causal_padding(k, d)
    for j in range(k):
        y = H.causal_conv(x, _tap(4, 4, k, j), torch.zeros(4), dilation=d)
        shift = pad - j * d
        ref = torch.cat([torch.zeros(1, 4, shift), x[:, :, :20 - shift]], dim=2)
        torch.testing.assert_close(y, ref)


def test_right_conv_looks_ahead_with_context():
    """Right type (k = 5, 4 frames ahead): tap j reads x[t + j]; with a cache, the cache
    frames replace the zero padding."""
    x = torch.randn(1, 4, 12, generator=torch.Generator().manual_seed(2))
    y = H.causal_conv(x, _tap(4, 4, 5, 4), torch.zeros(4), right=True)
    torch.testing.assert_close(y, torch.cat([x[:, :, 4:], torch.zeros(1, 4, 4)], dim=2))
    yc = H.causal_conv(x[:, :, :8], _tap(4, 4, 5, 4), torch.zeros(4), right=True,
                       cache=x[:, :, 8:])
    torch.testing.assert_close(yc, x[:, :, 4:])


def test_down_and_up_convolutions():
    x = torch.randn(1, 4, 30, generator=torch.Generator().manual_seed(3))
    # stride 3, kernel 6: tap 2 reads x[3 t] (2 zeros of left padding)
    y = H.down_conv(x, _tap(4, 4, 6, 2), torch.zeros(4), 3)
    assert y.shape[2] == (30 + 2 - 6) // 3 + 1
    torch.testing.assert_close(y, x[:, :, 0::3][:, :, :y.shape[2]])
    # nearest upsampling by 5, kernel 11: the last tap reads x[t // 5]
    u = H.up_conv(x, _tap(4, 4, 11, 10), torch.zeros(4), 5)
    torch.testing.assert_close(u, x.repeat_interleave(5, dim=2))


def test_snake_closed_form():
    x = torch.tensor([[[0.0, math.pi / 2, 1.0]]])
    a = torch.tensor([1.0])
    ref = torch.tensor([[[0.0, math.pi / 2 + 1.0, 1.0 + math.sin(1.0) ** 2]]])
    torch.testing.assert_close(H.snake(x, a), ref)


def test_stft_istft_reconstruct(fcv):
    dims = fcv.synthetic.HiFTDims()
    x = torch.randn(1, 480 * 7, generator=torch.Generator().manual_seed(4))
    re, im = H.stft(x, dims)
    assert re.shape == (1, 9, 480 * 7 // 4 + 1)
    mag, ph = torch.sqrt(re ** 2 + im ** 2), torch.atan2(im, re)
    # istft takes (magnitude, phase); sin(phase) inside the vocoder is a separate step
    y = H.istft(mag, ph, dims)
    torch.testing.assert_close(y, x, rtol=1e-4, atol=1e-4)


def test_source_for_constant_f0(fcv):
    """F0 = 200 Hz everywhere, zero noise table: every frame is voiced, harmonic h advances
    480 * (200 (h+1) / 24000 mod 1) cycles per frame, and within a frame the sine is held."""
    dims = fcv.synthetic.HiFTDims()
    H_ = dims.nb_harmonics + 1
    T = 6
    sd = {"m_source.l_linear.weight": torch.zeros(1, H_), "m_source.l_linear.bias": torch.zeros(1)}
    sd["m_source.l_linear.weight"][0, 1] = 1.0  # pick harmonic 2
    buf = {"rand_ini": torch.zeros(1, H_), "sine_waves": torch.zeros(1, T * 480, H_)}
    s = H.source(sd, torch.full((1, T), 200.0), buf, dims)[0, 0]
    rad = (200.0 * 2 / 24000) % 1
    for d in range(T):
        phase = 2 * math.pi * (d + 1) * rad * 480
        want = math.tanh(0.1 * math.sin(phase))
        frame = s[d * 480:(d + 1) * 480]
        assert torch.allclose(frame, torch.full_like(frame, want), atol=2e-4)
