"""CPU checks that pin the Flow front-end oracle (oracle/frontend_oracle.py).

``frontend.npz`` holds outputs of the reference's own ``PreLookaheadLayer``
(upsample_encoder.py:55-92).  The embedding lookup, the mask, ``F.normalize`` + ``Linear`` and
the prompt copy are torch primitives in the reference (flashinfer_flow.py:93-115,144-151); they
are pinned here by closed forms and invariants (unit-norm inputs, scale invariance, receptive
field, residual identity, exact copies).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import frontend_oracle as F

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def golden(fcv):
    z = np.load(GOLDEN / "frontend.npz")
    dims = fcv.synthetic.FlowDims(vocab=int(z["vocab"]), channels=int(z["channels"]))
    sd = fcv.synthetic.random_flow_state_dict(dims, seed=int(z["weight_seed"]))
    return z, sd


def _la(sd):
    return [sd[f"pre_lookahead_layer.{k}"] for k in ("conv1.weight", "conv1.bias",
                                                    "conv2.weight", "conv2.bias")]


def test_golden_inputs_regenerate(golden):
    """The fixture's embedded inputs equal masked embedding rows of the seeded table."""
    z, sd = golden
    lengths = [int(v) for v in z["lengths"]]
    x = F.embed_tokens(sd["input_embedding.weight"], torch.from_numpy(z["tokens"]), lengths)
    assert torch.equal(x, torch.from_numpy(z["x"]))


def test_pre_lookahead_matches_reference_layer(golden):
    z, sd = golden
    x = torch.from_numpy(z["x"])
    out = F.pre_lookahead(x, *_la(sd))
    torch.testing.assert_close(out, torch.from_numpy(z["out_batch"]), rtol=1e-5, atol=1e-5)
    split = int(z["ctx_split"])
    ctx = F.pre_lookahead(x[0:1, :split], *_la(sd), context=x[0:1, split:13])
    torch.testing.assert_close(ctx, torch.from_numpy(z["ctx_out"]), rtol=1e-5, atol=1e-5)


def test_padded_batch_equals_documents_alone(golden):
    """Valid frames of the padded, masked batch equal each document run alone: the property
    that lets the front-end work on packed documents."""
    z, _ = golden
    for b, n in enumerate(z["lengths"]):
        np.testing.assert_allclose(z["out_batch"][b, :n], z["out_single"][b, :n], rtol=1e-5,
                                   atol=1e-5)


def test_context_equals_lookahead_over_the_full_document(golden):
    """With the last three tokens as context, the outputs equal the first frames of the
    finalized document: context only replaces the zero padding."""
    z, sd = golden
    split = int(z["ctx_split"])
    full = torch.from_numpy(z["out_single"][0:1, :13])
    np.testing.assert_allclose(z["ctx_out"][0], full[0, :split].numpy(), rtol=1e-5, atol=1e-5)


def test_receptive_field_is_two_back_three_ahead():
    """conv1 reads frames t..t+3, conv2 reads conv1 at t-2..t: output t depends on inputs
    t-2..t+3 only; perturbing input u moves outputs u-3..u+2 only."""
    g = torch.Generator().manual_seed(3)
    C, T, u = 64, 20, 9
    w1, b1 = torch.randn(C, 80, 4, generator=g) * 0.1, torch.randn(C, generator=g)
    w2, b2 = torch.randn(80, C, 3, generator=g) * 0.1, torch.randn(80, generator=g)
    x = torch.randn(1, T, 80, generator=g, dtype=torch.float32)
    y0 = F.pre_lookahead(x, w1, b1, w2, b2)
    x2 = x.clone()
    x2[0, u] += 1.0
    diff = (F.pre_lookahead(x2, w1, b1, w2, b2) - y0).abs().amax(-1)[0]
    moved = torch.nonzero(diff > 1e-6).flatten().tolist()
    assert moved == list(range(u - 3, u + 3))


def test_residual_identity_and_bias():
    """Zero conv2 weights: output = input + conv2 bias, whatever conv1 does."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 7, 80, generator=g)
    b2 = torch.randn(80, generator=g)
    y = F.pre_lookahead(x, torch.randn(32, 80, 4, generator=g), torch.randn(32, generator=g),
                        torch.zeros(80, 32, 3), b2)
    torch.testing.assert_close(y, x + b2, rtol=0, atol=0)


def test_single_tap_conv1_is_a_shift():
    """conv1 with only tap 2 set to the identity and conv2 with only its last tap the identity
    gives leaky_relu(x[t+2]) + x[t] (x[t+2] = 0 past the end)."""
    x = torch.randn(1, 9, 80, generator=torch.Generator().manual_seed(8))
    w1 = torch.zeros(80, 80, 4)
    w1[:, :, 2] = torch.eye(80)
    w2 = torch.zeros(80, 80, 3)
    w2[:, :, 2] = torch.eye(80)
    y = F.pre_lookahead(x, w1, torch.zeros(80), w2, torch.zeros(80))
    shifted = torch.cat([x[:, 2:], torch.zeros(1, 2, 80)], dim=1)
    ref = torch.where(shifted > 0, shifted, 0.01 * shifted) + x
    torch.testing.assert_close(y, ref, rtol=1e-6, atol=1e-6)


def test_embedding_clamps_negative_ids_and_masks_padding():
    table = torch.arange(5 * 80, dtype=torch.float32).reshape(5, 80)
    tokens = torch.tensor([[-3, 4, 1], [2, 0, 0]])
    x = F.embed_tokens(table, tokens, [3, 1])
    assert torch.equal(x[0, 0], table[0]) and torch.equal(x[0, 1], table[4])
    assert torch.equal(x[1, 0], table[2]) and not x[1, 1:].any()


def test_speaker_projection_closed_forms():
    g = torch.Generator().manual_seed(9)
    w, b = torch.randn(80, 192, generator=g), torch.randn(80, generator=g)
    x = torch.randn(4, 192, generator=g, dtype=torch.float64).float()
    unit = x / x.norm(dim=1, keepdim=True)
    torch.testing.assert_close(F.speaker_projection(unit, w, b), unit @ w.T + b, rtol=1e-5,
                               atol=1e-5)
    torch.testing.assert_close(F.speaker_projection(7.5 * x, w, b), F.speaker_projection(x, w, b),
                               rtol=1e-5, atol=1e-5)
    # a zero x-vector divides by eps = 1e-12 and projects to the bias alone
    torch.testing.assert_close(F.speaker_projection(torch.zeros(1, 192), w, b), b[None])


def test_flow_inputs_packing(fcv):
    """mu repeats each token's row token_mel_ratio times, Mel lengths are 2 x tokens, the
    condition holds the prompt then zeros, and padding past a document never leaks in."""
    dims = fcv.synthetic.FlowDims(vocab=50, channels=128)
    sd = fcv.synthetic.random_flow_state_dict(dims, seed=1)
    g = torch.Generator().manual_seed(2)
    toks = [[1, 2, 3, 4, 5, 6], [7, -1, 9]]
    prompts = [torch.randn(1, 4, 80, generator=g), torch.randn(1, 0, 80, generator=g)]
    xvec = torch.randn(2, 192, generator=g)
    mu, cond, spks, mel, plen = F.flow_inputs(sd, toks, prompts, xvec)
    assert mel == [12, 6] and plen == [4, 0] and mu.shape == (2, 80, 12)
    torch.testing.assert_close(mu[:, :, 0::2], mu[:, :, 1::2], rtol=0, atol=0)
    assert torch.equal(cond[0, :, :4], prompts[0][0].T) and not cond[0, :, 4:].any()
    assert not cond[1].any()
    alone = F.streaming_token_features(sd, toks[1], finalize=True)
    torch.testing.assert_close(mu[1, :, :6].T, alone[0], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(spks, F.speaker_projection(xvec, sd["spk_embed_affine_layer.weight"],
                                                          sd["spk_embed_affine_layer.bias"]))


def test_streaming_features_with_context(fcv, golden):
    """Non-final streams emit (len - 3) x ratio rows equal to the context form of the layer."""
    z, sd = golden
    toks = [int(v) for v in z["tokens"][0, :13]]
    out = F.streaming_token_features(sd, toks, finalize=False)
    assert out.shape == (1, 20, 80)
    ref = torch.from_numpy(z["ctx_out"]).repeat_interleave(2, dim=1)
    torch.testing.assert_close(out, ref, rtol=1e-5, atol=1e-5)
