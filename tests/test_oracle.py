"""Pin the fp32 CPU oracle: golden vectors from the reference, closed forms, brute force on
tiny inputs and the invariants the reference's own tests rely on."""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import dit_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


def _golden(name):
    return dict(np.load(GOLDEN / name, allow_pickle=False))


def _weights(fcv, g):
    dims = fcv.synthetic.DiTDims(dim=int(g["dim"]), depth=int(g["depth"]), heads=int(g["heads"]))
    return fcv.synthetic.random_state_dict(dims, seed=int(g["weight_seed"]),
                                           gate_bias=float(g["gate_bias"]))


# ---- golden vectors written by tests/golden/make_golden.py from the reference DiT ----------


@pytest.mark.parametrize("name", ["tiny_dit.npz", "block1024.npz"])
@pytest.mark.parametrize("streaming", [False, True])
def test_oracle_matches_reference_golden(fcv, name, streaming):
    g = _golden(name)
    sd = _weights(fcv, g)
    t = {k: torch.from_numpy(g[k]) for k in ("x", "mask", "mu", "t", "spks", "cond")}
    out = O.dit_forward(sd, t["x"], t["mask"], t["mu"], t["t"], t["spks"], t["cond"],
                        streaming=streaming, heads=int(g["heads"]), chunk_size=int(g["chunk"]))
    ref = torch.from_numpy(g["out_stream" if streaming else "out_full"])
    assert out.shape == ref.shape
    torch.testing.assert_close(out, ref, rtol=1e-4, atol=1e-4)


def test_oracle_solver_matches_reference_golden(fcv):
    g = _golden("tiny_dit.npz")
    sd = _weights(fcv, g)
    t = {k: torch.from_numpy(g[k]) for k in ("x", "mask", "mu", "spks", "cond")}
    est = lambda x, mask, mu, tt, spks, cond, streaming: O.dit_forward(
        sd, x, mask, mu, tt, spks, cond, streaming=streaming, heads=int(g["heads"]),
        chunk_size=int(g["chunk"]))
    sample = O.solve_euler_batched(est, t["x"], t["mu"], t["mask"], t["spks"], t["cond"],
                                   n_steps=int(g["euler_steps"]), cfg_rate=float(g["euler_cfg"]))
    torch.testing.assert_close(sample, torch.from_numpy(g["euler_sample"]), rtol=1e-4, atol=1e-4)


# ---- closed forms --------------------------------------------------------------------------


def test_sinusoid_closed_form():
    emb = O.sinus_position_embedding(torch.tensor([0.0, 0.5, 1.0]))
    assert emb.shape == (3, 256)
    torch.testing.assert_close(emb[0, :128], torch.zeros(128))
    torch.testing.assert_close(emb[0, 128:], torch.ones(128))
    # frequency i is 10000^(-i/127); argument is 1000 * t * f_i
    for t, row in ((0.5, 1), (1.0, 2)):
        for i in (0, 1, 64, 127):
            f = 10000.0 ** (-i / 127.0)
            assert abs(emb[row, i].item() - math.sin(1000 * t * f)) < 2e-3
            assert abs(emb[row, 128 + i].item() - math.cos(1000 * t * f)) < 2e-3


def test_cosine_schedule_closed_form():
    span = O.cosine_schedule(10)
    expect = torch.tensor([1 - math.cos(k * math.pi / 20) for k in range(11)], dtype=torch.float32)
    torch.testing.assert_close(span, expect, rtol=0, atol=1e-6)


def test_layer_norm_matches_library():
    x = torch.randn(7, 1024) * 50 + 300
    torch.testing.assert_close(O.layer_norm(x), F.layer_norm(x, (1024,), eps=1e-6),
                               rtol=1e-4, atol=1e-4)


def test_activations_match_library():
    x = torch.linspace(-30, 30, 2001)
    torch.testing.assert_close(O.gelu_tanh(x), F.gelu(x, approximate="tanh"), rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(O.mish(x), F.mish(x), rtol=1e-5, atol=1e-5)


# ---- RoPE invariants -------------------------------------------------------------------------


def test_rotary_known_values_and_invariants():
    freqs = O.rotary_freqs(torch.arange(6), 64)
    x = torch.randn(6, 1024)
    y = O.apply_rotary(x, freqs)
    # position 0 is the identity; columns past head 0 never rotate
    torch.testing.assert_close(y[0], x[0])
    torch.testing.assert_close(y[:, 64:], x[:, 64:])
    # each interleaved pair keeps its norm
    px, py = x[:, :64].reshape(6, 32, 2), y[:, :64].reshape(6, 32, 2)
    torch.testing.assert_close(px.norm(dim=-1), py.norm(dim=-1), rtol=1e-5, atol=1e-5)
    # pair 0 at position 1 rotates (1, 0) to (cos 1, sin 1): counter-clockwise, angle p*1
    e = torch.zeros(2, 1024)
    e[:, 0] = 1.0
    r = O.apply_rotary(e, O.rotary_freqs(torch.arange(2), 64))
    assert abs(r[1, 0].item() - math.cos(1.0)) < 1e-6 and abs(r[1, 1].item() - math.sin(1.0)) < 1e-6
    # pair i rotates by p * 10000^(-2i/64)
    for i in (1, 7, 31):
        e = torch.zeros(4, 1024)
        e[:, 2 * i] = 1.0
        r = O.apply_rotary(e, O.rotary_freqs(torch.arange(4), 64))
        ang = 3 * 10000.0 ** (-2 * i / 64)
        assert abs(r[3, 2 * i].item() - math.cos(ang)) < 1e-5
        assert abs(r[3, 2 * i + 1].item() - math.sin(ang)) < 1e-5


def test_rotary_composes():
    # R(p) then R(q) == R(p+q) on the rotated pairs
    x = torch.randn(1, 1024)
    p, q = 5, 11
    a = O.apply_rotary(O.apply_rotary(x, O.rotary_freqs(torch.tensor([p]), 64)),
                       O.rotary_freqs(torch.tensor([q]), 64))
    b = O.apply_rotary(x, O.rotary_freqs(torch.tensor([p + q]), 64))
    torch.testing.assert_close(a, b, rtol=1e-4, atol=1e-4)


# ---- masks ------------------------------------------------------------------------------------


def test_chunk_mask_reference_docstring_example():
    # mask.py:147-152 documents subsequent_chunk_mask(4, 2)
    expect = torch.tensor([[1, 1, 0, 0], [1, 1, 0, 0], [1, 1, 1, 1], [1, 1, 1, 1]], dtype=torch.bool)
    assert torch.equal(O.subsequent_chunk_mask(4, 2), expect)


def test_attention_mask_padding_and_chunks():
    mask = torch.zeros(2, 1, 6)
    mask[0, 0, :6] = 1
    mask[1, 0, :4] = 1
    full = O.attention_mask(mask, streaming=False)
    assert full.shape == (2, 1, 6, 6)
    assert torch.equal(full[1, 0, 5], torch.tensor([1, 1, 1, 1, 0, 0], dtype=torch.bool))
    st = O.attention_mask(mask, streaming=True, chunk_size=2)
    # key k visible iff k//2 <= q//2 and k < length
    for b, n in ((0, 6), (1, 4)):
        for q in range(6):
            for k in range(6):
                assert bool(st[b, 0, q, k]) == (k < n and k // 2 <= q // 2)
    # an all-False row is forced True (mask.py:232-234)
    empty = O.attention_mask(torch.zeros(1, 1, 3), streaming=False)
    assert empty.all()


# ---- brute force on tiny inputs -----------------------------------------------------------


def test_causal_conv_brute_force():
    torch.manual_seed(0)
    C, G, K, T = 32, 16, 5, 9
    sd = {"input_embed.conv_pos_embed.conv1.0.weight": torch.randn(C, C // G, K),
          "input_embed.conv_pos_embed.conv1.0.bias": torch.randn(C),
          "input_embed.conv_pos_embed.conv2.0.weight": torch.randn(C, C // G, K),
          "input_embed.conv_pos_embed.conv2.0.bias": torch.randn(C)}
    h = torch.randn(1, T, C)

    def conv(x, w, b):  # x [T, C]
        y = torch.zeros(T, C)
        cpg = C // G
        for t in range(T):
            for co in range(C):
                g = co // cpg
                acc = b[co].item()
                for j in range(K):
                    src = t - (K - 1) + j
                    if src < 0:
                        continue
                    for ci in range(cpg):
                        acc += w[co, ci, j].item() * x[src, g * cpg + ci].item()
                y[t, co] = acc
        return O.mish(y)

    pre = "input_embed.conv_pos_embed."
    brute = conv(conv(h[0], sd[pre + "conv1.0.weight"], sd[pre + "conv1.0.bias"]),
                 sd[pre + "conv2.0.weight"], sd[pre + "conv2.0.bias"])
    ours = O.causal_conv_position_embedding(sd, h, kernel_size=K, groups=G)[0]
    torch.testing.assert_close(ours, brute, rtol=1e-4, atol=1e-4)


def test_attention_brute_force(fcv):
    dims = fcv.synthetic.DiTDims(dim=128, depth=1, heads=2)
    sd = fcv.synthetic.random_state_dict(dims, seed=3, std=0.2)
    T = 7
    x = torch.randn(1, T, 128)
    freqs = O.rotary_freqs(torch.arange(T), 64)
    mask = O.attention_mask(torch.ones(1, 1, T), streaming=True, chunk_size=3)
    out = O.attention(sd, 0, x, mask, freqs, heads=2)
    p = "transformer_blocks.0.attn."
    q = O.apply_rotary(F.linear(x, sd[p + "to_q.weight"], sd[p + "to_q.bias"]), freqs)[0]
    k = O.apply_rotary(F.linear(x, sd[p + "to_k.weight"], sd[p + "to_k.bias"]), freqs)[0]
    v = F.linear(x, sd[p + "to_v.weight"], sd[p + "to_v.bias"])[0]
    o = torch.zeros(T, 128)
    for h in range(2):
        cols = slice(64 * h, 64 * h + 64)
        for i in range(T):
            scores = [(q[i, cols] @ k[j, cols]).item() / 8.0 if j // 3 <= i // 3 else -math.inf
                      for j in range(T)]
            m = max(scores)
            w = [math.exp(s - m) for s in scores]
            z = sum(w)
            o[i, cols] = sum(w[j] / z * v[j, cols] for j in range(T))
    brute = F.linear(o, sd[p + "to_out.0.weight"], sd[p + "to_out.0.bias"])
    torch.testing.assert_close(out[0], brute, rtol=1e-4, atol=1e-4)


# ---- invariants ---------------------------------------------------------------------------


def _tiny(fcv, seed=1, gate_bias=0.5, depth=2):
    dims = fcv.synthetic.DiTDims(dim=128, depth=depth, heads=2)
    return fcv.synthetic.random_state_dict(dims, seed=seed, gate_bias=gate_bias)


def _padded_inputs(lengths, T, seed=0):
    g = torch.Generator().manual_seed(seed)
    B = len(lengths)
    x, mu, cond = (torch.randn(B, 80, T, generator=g) for _ in range(3))
    spks = torch.randn(B, 80, generator=g)
    t = torch.rand(B, generator=g)
    mask = torch.zeros(B, 1, T)
    for b, n in enumerate(lengths):
        mask[b, 0, :n] = 1
    return x, mask, mu, t, spks, cond


@pytest.mark.parametrize("streaming", [False, True])
def test_packed_equals_padded(fcv, streaming):
    sd = _tiny(fcv)
    lengths, T = [23, 9, 16], 23
    x, mask, mu, t, spks, cond = _padded_inputs(lengths, T)
    padded = O.dit_forward(sd, x, mask, mu, t, spks, cond, streaming=streaming, heads=2, chunk_size=5)
    packed = O.dit_forward_packed(sd, O.pack(x, lengths), O.pack(mu, lengths), O.pack(cond, lengths),
                                  spks, t, lengths, streaming=streaming, heads=2, chunk_size=5)
    torch.testing.assert_close(O.pack(padded, lengths), packed, rtol=1e-4, atol=1e-4)


def test_streaming_prefix_stability(fcv):
    # reference Gate A (tests/gpu/test_flashinfer_streaming_estimator.py:58-89), chunk 5
    sd = _tiny(fcv)
    x, mask, mu, t, spks, cond = _padded_inputs([20], 20)
    t = t[:1]
    cut = lambda a, n: a[..., :n].contiguous()
    old = O.dit_forward(sd, cut(x, 17), cut(mask, 17), cut(mu, 17), t, spks, cut(cond, 17),
                        streaming=True, heads=2, chunk_size=5)
    new = O.dit_forward(sd, x, mask, mu, t, spks, cond, streaming=True, heads=2, chunk_size=5)
    torch.testing.assert_close(old[..., :15], new[..., :15], rtol=0, atol=1e-5)
    off_old = O.dit_forward(sd, cut(x, 17), cut(mask, 17), cut(mu, 17), t, spks, cut(cond, 17),
                            streaming=False, heads=2)
    off_new = O.dit_forward(sd, x, mask, mu, t, spks, cond, streaming=False, heads=2)
    # full attention lets the 3 extra frames reach every earlier frame
    assert (off_old[..., :15] - off_new[..., :15]).abs().max() > 1e-3


def test_zero_gates_make_blocks_identity(fcv):
    sd = _tiny(fcv, depth=3, gate_bias=0.0)
    for i in range(3):
        w = sd[f"transformer_blocks.{i}.attn_norm.linear.weight"].view(6, 128, 128)
        b = sd[f"transformer_blocks.{i}.attn_norm.linear.bias"].view(6, 128)
        for c in (2, 5):
            w[c].zero_()
            b[c].zero_()
    shallow = {k: v for k, v in sd.items() if not k.startswith("transformer_blocks.")}
    x, mask, mu, t, spks, cond = _padded_inputs([11], 11)
    deep = O.dit_forward(sd, x, mask, mu, t, spks, cond, heads=2)
    # depth 0: input embedding -> final AdaLN -> proj_out
    temb = O.timestep_embedding(shallow, t)
    h = O.input_embedding(shallow, x.transpose(1, 2), cond.transpose(1, 2), mu.transpose(1, 2), spks)
    scale, shift = O.final_modulation(shallow, temb)
    h = O.layer_norm(h) * (1 + scale)[:, None] + shift[:, None]
    flat = F.linear(h, shallow["proj_out.weight"], shallow["proj_out.bias"]).transpose(1, 2)
    torch.testing.assert_close(deep, flat, rtol=1e-5, atol=1e-5)


def test_euler_constant_velocity_closed_form():
    B, T = 2, 5
    noise = torch.randn(B, 80, T)
    a, b = torch.randn(B, 80, T), torch.randn(B, 80, T)
    est = lambda x, mask, mu, t, spks, cond, streaming: torch.cat([a, b])
    out = O.solve_euler_batched(est, noise, torch.zeros(B, 80, T), torch.ones(B, 1, T),
                                torch.zeros(B, 80), torch.zeros(B, 80, T), n_steps=10, cfg_rate=0.7)
    # sum of the steps telescopes to span[-1] - span[0] = 1
    torch.testing.assert_close(out, noise + (1.7 * a - 0.7 * b), rtol=1e-5, atol=1e-5)


def test_euler_cfg_zero_is_conditional_only(fcv):
    sd = _tiny(fcv)
    x, mask, mu, t, spks, cond = _padded_inputs([12], 12)
    est = lambda xx, m, mm, tt, ss, cc, st: O.dit_forward(sd, xx, m, mm, tt, ss, cc, st, heads=2)
    cfg0 = O.solve_euler_batched(est, x, mu, mask, spks, cond, n_steps=3, cfg_rate=0.0)
    # plain Euler on the conditional estimator alone
    span = O.cosine_schedule(3)
    y = x.clone()
    for k in range(3):
        v = O.dit_forward(sd, y, mask, mu, torch.full((1,), float(span[k])), spks, cond, heads=2)
        y = y + (span[k + 1] - span[k]) * v
    torch.testing.assert_close(cfg0, y, rtol=1e-4, atol=1e-4)
