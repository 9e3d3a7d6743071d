"""GPU parity of the Flow front-end (include/fcv_flow.h) against the oracle and closed forms, and
the end-to-end flow entry points.

Tolerances: the front-end computes in fp32 on the fp32 matrix cores, so token features match
the fp32 oracle to rel-L2 <= 1e-5; the speaker projection to 1e-5; the prompt copy is exact; a
document's features do not depend on the batch (bit-exact).  End to end (front-end + 10-step
CFG solve) the Mel matches the fp32 oracle pipeline to rel-L2 <= 2e-2.
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from oracle import dit_oracle as O
from oracle import frontend_oracle as F
from tests.gpu_helpers import make_estimator, rel_l2, say

pytestmark = pytest.mark.gpu

FEAT_TOL = 1e-5


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _frontend(fcv, dims, sd):
    fe = fcv.FlowFrontEnd(vocab_size=dims.vocab, channels=dims.channels,
                          pre_lookahead_len=dims.lookahead, device="cuda:0")
    fe.load_reference_state_dict(sd)
    fe.finalize_weights()
    return fe


@pytest.fixture(scope="module")
def full_fe(fcv):
    """Front-end at the builders.py shapes (vocab 6561, 1024 channels) with seeded weights."""
    dims = fcv.synthetic.FlowDims()
    sd = fcv.synthetic.random_flow_state_dict(dims, seed=7)
    return sd, _frontend(fcv, dims, sd)


def _oracle_rows(sd, token_list, finalize=None):
    """Oracle packed mu rows: each document alone (the reference's streaming form)."""
    fin = finalize or [True] * len(token_list)
    return torch.cat([F.streaming_token_features(sd, t, f)[0] for t, f in zip(token_list, fin)])


def test_token_features_closed_form(fcv):
    """conv1 = identity from tap 2 into channels 0..79 (the rest zero), conv2 = identity from
    its last tap: every Mel row pair is leaky_relu(e(t+2)) + e(t), zero past the document."""
    dims = fcv.synthetic.FlowDims(vocab=50, channels=128)
    sd = fcv.synthetic.random_flow_state_dict(dims, seed=3)
    w1 = torch.zeros(128, 80, 4)
    w1[:80, :, 2] = torch.eye(80)
    w2 = torch.zeros(80, 128, 3)
    w2[:, :80, 2] = torch.eye(80)
    sd.update({"pre_lookahead_layer.conv1.weight": w1,
               "pre_lookahead_layer.conv1.bias": torch.zeros(128),
               "pre_lookahead_layer.conv2.weight": w2,
               "pre_lookahead_layer.conv2.bias": torch.zeros(80)})
    fe = _frontend(fcv, dims, sd)
    lengths = [13, 6, 1, 70]
    g = torch.Generator().manual_seed(4)
    toks = [torch.randint(0, 50, (n,), generator=g).tolist() for n in lengths]
    say(f"[fe closed form] lengths {lengths}")
    mu, mel = fe.token_features(toks)
    assert mel == [2 * n for n in lengths]
    mu = mu.cpu()
    table = sd["input_embedding.weight"]
    ref = []
    for t in toks:
        e = table[torch.tensor(t)]
        ahead = torch.cat([e[2:], torch.zeros(2, 80)])[:len(t)]
        ref.append(torch.where(ahead > 0, ahead, 0.01 * ahead) + e)
    ref = torch.cat(ref).repeat_interleave(2, dim=0)
    torch.testing.assert_close(mu, ref, rtol=1e-6, atol=1e-6)


def test_context_rows_equal_finalized_prefix(fcv, full_fe):
    """A non-final stream's rows equal the first rows of the same stream finalized (context
    tokens stand in for the zero padding), bit for bit."""
    _, fe = full_fe
    g = torch.Generator().manual_seed(5)
    toks = [torch.randint(0, 6561, (n,), generator=g).tolist() for n in (4, 13, 150)]
    say("[fe context]")
    part, mel_p = fe.token_features(toks, [False] * 3)
    full, mel_f = fe.token_features(toks)
    op = of = 0
    for mp, mf in zip(mel_p, mel_f):
        assert mp == mf - 6
        assert torch.equal(part[op:op + mp], full[of:of + mp])
        op, of = op + mp, of + mf


def test_token_features_ragged_full_size(fcv, full_fe):
    """Ragged documents (1 token up to 777, across tile edges) with negative ids, against the
    oracle's padded-batch front-end (flashinfer_flow.py:144-151)."""
    sd, fe = full_fe
    lengths = [1, 2, 3, 4, 5, 63, 64, 65, 200, 777]
    g = torch.Generator().manual_seed(11)
    toks = [torch.randint(-2, 6561, (n,), generator=g).tolist() for n in lengths]
    say(f"[fe ragged] lengths {lengths}")
    mu, mel = fe.token_features(toks)
    ref_mu, _, _, ref_mel, _ = F.flow_inputs(sd, toks, [torch.zeros(1, 0, 80)] * len(toks),
                                             torch.ones(len(toks), 192))
    assert mel == ref_mel
    ref = torch.cat([ref_mu[b, :, :m].T for b, m in enumerate(mel)])
    err = rel_l2(mu.cpu(), ref)
    say(f"[fe ragged] rel_l2 {err:.2e}, max abs {float((mu.cpu() - ref).abs().max()):.2e}")
    assert err <= FEAT_TOL


def test_token_features_streaming_mix(fcv, full_fe):
    """Final and non-final streams in one call (_streaming_token_features per stream)."""
    sd, fe = full_fe
    lengths, fin = [4, 4, 50, 129, 1], [True, False, False, True, True]
    g = torch.Generator().manual_seed(12)
    toks = [torch.randint(0, 6561, (n,), generator=g).tolist() for n in lengths]
    say("[fe stream] finalize mix")
    mu, mel = fe.token_features(toks, fin)
    assert mel == [2 * (n - (0 if f else 3)) for n, f in zip(lengths, fin)]
    err = rel_l2(mu.cpu(), _oracle_rows(sd, toks, fin))
    say(f"[fe stream] rel_l2 {err:.2e}")
    assert err <= FEAT_TOL


def test_token_features_batch_invariant(fcv, full_fe):
    """A document's rows are bit-identical alone and packed between other documents."""
    _, fe = full_fe
    g = torch.Generator().manual_seed(13)
    toks = [torch.randint(0, 6561, (n,), generator=g).tolist() for n in (70, 333, 5, 129)]
    say("[fe invariance]")
    batch, mel = fe.token_features(toks)
    off = 0
    for t, m in zip(toks, mel):
        alone, _ = fe.token_features([t])
        assert torch.equal(alone, batch[off:off + m])
        off += m


def test_speaker_projection(fcv, full_fe):
    sd, fe = full_fe
    g = torch.Generator().manual_seed(14)
    x = torch.randn(6, 192, generator=g) * torch.tensor([1, 3, 0.01, 100, 1, 1])[:, None]
    x[4] = 0.0
    say("[fe speaker]")
    out = fe.speaker(x).cpu()
    ref = F.speaker_projection(x, sd["spk_embed_affine_layer.weight"],
                               sd["spk_embed_affine_layer.bias"])
    err = rel_l2(out, ref)
    say(f"[fe speaker] rel_l2 {err:.2e}")
    assert err <= FEAT_TOL
    torch.testing.assert_close(out[4], sd["spk_embed_affine_layer.bias"])


def test_prompt_condition_exact(fcv, full_fe):
    """Prompt rows copied bit-exactly, zeros after; empty prompts and a prompt as long as the
    document (_copy_prompt_features)."""
    _, fe = full_fe
    g = torch.Generator().manual_seed(15)
    mel = [10, 8, 12, 4]
    plens = [0, 5, 12, 4]
    prompts = [torch.randn(1, p, 80, generator=g) for p in plens]
    say("[fe prompt]")
    cond, pl = fe.prompt_condition(prompts, mel)
    assert pl == plens
    sd = fcv.synthetic.random_flow_state_dict(fcv.synthetic.FlowDims(vocab=1, channels=128))
    _, ref, _, ref_mel, _ = F.flow_inputs(sd, [[0] * (m // 2) for m in mel], prompts,
                                          torch.ones(4, 192))
    assert ref_mel == mel
    ref_rows = torch.cat([ref[b, :, :m].T for b, m in enumerate(mel)])
    assert torch.equal(cond.cpu(), ref_rows)


def test_frontend_errors(fcv, full_fe):
    """The reference's failures: out-of-range ids (nn.Embedding IndexError), a non-final stream
    without tokens beyond its lookahead, mismatched finalize flags (ValueError)."""
    _, fe = full_fe
    with pytest.raises(IndexError):
        fe.token_features([[1, 2, 6561]])
    with pytest.raises(ValueError, match="lookahead"):
        fe.token_features([[1, 2, 3]], [False])
    with pytest.raises(ValueError, match="same length"):
        fe.token_features([[1, 2, 3, 4]], [False, True])
    with pytest.raises(ValueError, match="no tokens"):
        fe.token_features([[1, 2], []])


def test_flow_inference_batched_end_to_end(fcv):
    """Tokens -> Mel through the front-end and the packed 10-step CFG solve (2 DiT blocks at
    full width) against the oracle pipeline fed the same noise."""
    dims = fcv.synthetic.FlowDims()
    fsd = fcv.synthetic.random_flow_state_dict(dims, seed=31)
    fe = _frontend(fcv, dims, fsd)
    dsd = fcv.synthetic.random_state_dict(fcv.synthetic.DiTDims(depth=2), seed=32,
                                          gate_bias=0.5)
    est = make_estimator(fcv, dsd, depth=2)
    fe.decoder = SimpleNamespace(estimator=est, inference_cfg_rate=0.7)
    g = torch.Generator().manual_seed(33)
    token_list = [torch.randint(0, 6561, (n,), generator=g).tolist() for n in (40, 25, 61)]
    prompts = [torch.randn(1, p, 80, generator=g) for p in (20, 0, 30)]
    xvec = torch.randn(3, 192, generator=g)
    mel = [2 * len(t) for t in token_list]
    noise = torch.randn(3, 80, max(mel), generator=g)
    say("[fe e2e] GPU flow_inference_batched")
    out = fcv.flow_inference_batched(fe, token_list, prompts, xvec.cuda(), noise=noise.cuda())
    say("[fe e2e] oracle pipeline")
    mu, cond, spks, mel_ref, plens = F.flow_inputs(fsd, token_list, prompts, xvec)
    assert mel_ref == mel
    mask = torch.zeros(3, 1, max(mel))
    for b, m in enumerate(mel):
        mask[b, 0, :m] = 1

    def oracle_est(x, mask, mu, t, spks, cond, streaming):
        return O.dit_forward(dsd, x, mask, mu, t, spks, cond, streaming=streaming)

    ref = O.solve_euler_batched(oracle_est, noise, mu, mask, spks, cond, n_steps=10, cfg_rate=0.7)
    for b in range(3):
        want = ref[b:b + 1, :, plens[b]:mel[b]]
        assert out[b].shape == want.shape
        err = rel_l2(out[b].cpu(), want)
        say(f"[fe e2e] request {b} mel rel_l2 {err:.2e}")
        assert err <= 2e-2
