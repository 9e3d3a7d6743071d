"""CPU checks that pin the Flow front-end oracle (oracle/frontend_oracle.py) by closed forms,
invariants and the reference's own layer.

``tests/golden/prelookahead.npz`` holds the outputs of the reference's ``PreLookaheadLayer``
(upsample_encoder.py:55-92, written by tests/golden/make_golden.py at the flow's shape with our
seeded weights): a finalized padded batch and the streaming form with a right context.
Beyond that, ``PreLookaheadLayer`` (upsample_encoder.py:55-92) is pinned piece by piece: the direction and
tap order of the lookahead convolution and the LeakyReLU slope (a one-tap identity conv1 gives
leaky_relu(x[t+2])), the causal left padding of conv2 (its last tap is the current frame; the
receptive field of output t is exactly t-2 .. t+3), the residual (zero conv2 gives x + b2), the
context form (context frames take the place of the zero padding, so a non-final stream's
outputs equal the first frames of the finalized stream) and the padded-batch form (valid
frames equal each document alone).  The embedding lookup with clamp and mask, ``F.normalize`` +
``Linear`` and the prompt copy (flashinfer_flow.py:93-115,144-151) are pinned by exact closed
forms.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

from oracle import frontend_oracle as F

GOLDEN = Path(__file__).resolve().parent / "golden"


def _weights(C=64, seed=3):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(C, 80, 4, generator=g) * 0.1, torch.randn(C, generator=g),
            torch.randn(80, C, 3, generator=g) * 0.1, torch.randn(80, generator=g))


def test_receptive_field_is_two_back_three_ahead():
    """conv1 reads frames t..t+3, conv2 reads conv1 at t-2..t: perturbing input u moves
    outputs u-3..u+2 only."""
    w = _weights()
    T, u = 20, 9
    x = torch.randn(1, T, 80, generator=torch.Generator().manual_seed(4))
    y0 = F.pre_lookahead(x, *w)
    x2 = x.clone()
    x2[0, u] += 1.0
    diff = (F.pre_lookahead(x2, *w) - y0).abs().amax(-1)[0]
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


def test_single_tap_identity_is_a_shifted_leaky_relu():
    """conv1 = identity on tap 2 only, conv2 = identity on its last tap only: the output is
    leaky_relu(x[t+2]) + x[t] with slope 0.01 and x[t+2] = 0 past the end."""
    x = torch.randn(1, 9, 80, generator=torch.Generator().manual_seed(8))
    w1 = torch.zeros(80, 80, 4)
    w1[:, :, 2] = torch.eye(80)
    w2 = torch.zeros(80, 80, 3)
    w2[:, :, 2] = torch.eye(80)
    y = F.pre_lookahead(x, w1, torch.zeros(80), w2, torch.zeros(80))
    shifted = torch.cat([x[:, 2:], torch.zeros(1, 2, 80)], dim=1)
    ref = torch.where(shifted > 0, shifted, 0.01 * shifted) + x
    torch.testing.assert_close(y, ref, rtol=1e-6, atol=1e-6)


def test_conv2_first_tap_reads_two_frames_back():
    """conv2 = identity on its first tap, conv1 = identity on tap 0: output t is
    leaky_relu(x[t-2]) + x[t], zero for t < 2 (left zero padding)."""
    x = torch.randn(1, 8, 80, generator=torch.Generator().manual_seed(9))
    w1 = torch.zeros(80, 80, 4)
    w1[:, :, 0] = torch.eye(80)
    w2 = torch.zeros(80, 80, 3)
    w2[:, :, 0] = torch.eye(80)
    y = F.pre_lookahead(x, w1, torch.zeros(80), w2, torch.zeros(80))
    back = torch.cat([torch.zeros(1, 2, 80), x[:, :-2]], dim=1)
    torch.testing.assert_close(y, torch.where(back > 0, back, 0.01 * back) + x, rtol=1e-6,
                               atol=1e-6)


def test_context_replaces_the_zero_padding():
    """With the last three frames as context, the outputs equal the first frames of the
    finalized sequence: context only stands in for the zero padding."""
    w = _weights(seed=10)
    x = torch.randn(1, 13, 80, generator=torch.Generator().manual_seed(11))
    full = F.pre_lookahead(x, *w)
    ctx = F.pre_lookahead(x[:, :10], *w, context=x[:, 10:])
    torch.testing.assert_close(ctx, full[:, :10], rtol=1e-5, atol=1e-5)


def test_padded_batch_equals_documents_alone():
    """Valid frames of the padded, masked batch equal each document run alone: the property
    that lets the front-end work on packed documents."""
    w = _weights(seed=12)
    table = torch.randn(30, 80, generator=torch.Generator().manual_seed(13))
    lengths = [13, 6, 1]
    tokens = torch.zeros(3, 13, dtype=torch.long)
    for b, n in enumerate(lengths):
        tokens[b, :n] = torch.randint(0, 30, (n,), generator=torch.Generator().manual_seed(b))
    batch = F.pre_lookahead(F.embed_tokens(table, tokens, lengths), *w)
    for b, n in enumerate(lengths):
        alone = F.pre_lookahead(table[tokens[b:b + 1, :n]], *w)
        # fp32 rounding differs between the batched and single convolution paths
        torch.testing.assert_close(batch[b:b + 1, :n], alone, rtol=1e-5, atol=1e-5)


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


def test_streaming_features_with_context(fcv):
    """Non-final streams emit (len - 3) x ratio rows, equal to the finalized stream's first
    rows (the context invariant through the whole streaming feature path)."""
    dims = fcv.synthetic.FlowDims(vocab=97, channels=128)
    sd = fcv.synthetic.random_flow_state_dict(dims, seed=21)
    toks = torch.randint(0, 97, (13,), generator=torch.Generator().manual_seed(3)).tolist()
    out = F.streaming_token_features(sd, toks, finalize=False)
    full = F.streaming_token_features(sd, toks, finalize=True)
    assert out.shape == (1, 20, 80) and full.shape == (1, 26, 80)
    torch.testing.assert_close(out, full[:, :20], rtol=1e-5, atol=1e-5)


def test_pre_lookahead_matches_reference_golden(fcv):
    """The oracle's pre_lookahead against the reference's PreLookaheadLayer on the same seeded
    weights (tests/golden/prelookahead.npz): the finalized padded batch (zero right pad) and a
    non-final stream whose last 3 frames arrive as right context."""
    g = dict(np.load(GOLDEN / "prelookahead.npz", allow_pickle=False))
    sd = fcv.synthetic.random_flow_state_dict(fcv.synthetic.FlowDims(), seed=int(g["weight_seed"]))
    w = [sd[f"pre_lookahead_layer.{k}"] for k in ("conv1.weight", "conv1.bias", "conv2.weight",
                                                  "conv2.bias")]
    look = int(g["lookahead"])
    out = F.pre_lookahead(torch.from_numpy(g["x"]), *w, look)
    ref = torch.from_numpy(g["out_final"])
    assert float((out - ref).abs().max()) <= 1e-5 * float(ref.abs().max())
    out = F.pre_lookahead(torch.from_numpy(g["x_stream"]), *w, look,
                          context=torch.from_numpy(g["context"]))
    ref = torch.from_numpy(g["out_context"])
    assert float((out - ref).abs().max()) <= 1e-5 * float(ref.abs().max())
