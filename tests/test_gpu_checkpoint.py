"""GPU checks of ``load_flow``: a flow built from a saved ``flow.pt`` gives bit-identical Mel to
one assembled by hand from the same tensors (the loader only routes weights), and the same Mel
as the oracle pipeline (front-end oracle + 10-step CFG Euler solve over the DiT oracle) run on
the state dict that was saved, within rel-L2 2e-2."""

from __future__ import annotations

import pytest
import torch

from oracle import dit_oracle as O
from oracle import frontend_oracle as F
from tests.gpu_helpers import make_estimator, rel_l2, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def test_load_flow_matches_hand_assembled_flow(fcv, tmp_path):
    syn = fcv.synthetic
    front = syn.random_flow_state_dict(syn.FlowDims(), seed=51)
    dit = syn.random_state_dict(syn.DiTDims(depth=2), seed=52, gate_bias=0.5)
    sd = dict(front)
    sd.update({"decoder.estimator." + k: v for k, v in dit.items()})
    path = tmp_path / "flow.pt"
    torch.save(sd, path)
    say("[ckpt] load_flow from flow.pt")
    loaded = fcv.load_flow(path)
    say("[ckpt] hand-assembled flow")
    fe = fcv.FlowFrontEnd(device="cuda:0")
    fe.load_reference_state_dict(front)
    fe.finalize_weights()
    fe.decoder = fcv.CFMDecoder(make_estimator(fcv, dit, depth=2))
    g = torch.Generator().manual_seed(53)
    toks = [torch.randint(0, 6561, (n,), generator=g).tolist() for n in (30, 47)]
    prompts = [torch.randn(1, 20, 80, generator=g), torch.randn(1, 10, 80, generator=g)]
    xvec = torch.randn(2, 192, generator=g).cuda()
    noise = torch.randn(2, 80, 94, generator=g).cuda()
    a = fcv.flow_inference_batched(loaded, toks, prompts, xvec, noise=noise)
    b = fcv.flow_inference_batched(fe, toks, prompts, xvec, noise=noise)
    assert all(torch.equal(x, y) for x, y in zip(a, b))

    say("[ckpt] oracle pipeline on the saved state dict")
    mu, cond, spks, mel, plens = F.flow_inputs(front, toks, prompts, xvec.cpu())
    mask = torch.zeros(2, 1, max(mel))
    for i, m in enumerate(mel):
        mask[i, 0, :m] = 1

    def oracle_est(x, mask, mu, t, spks, cond, streaming):
        return O.dit_forward(dit, x, mask, mu, t, spks, cond, streaming=streaming)

    ref = O.solve_euler_batched(oracle_est, noise.cpu(), mu, mask, spks, cond, n_steps=10,
                                cfg_rate=0.7)
    for i in range(2):
        want = ref[i:i + 1, :, plens[i]:mel[i]]
        assert a[i].shape == want.shape
        err = rel_l2(a[i].cpu(), want)
        say(f"[ckpt] request {i}: Mel rel_l2 vs oracle pipeline {err:.2e}")
        assert err <= 2e-2
    sa = fcv.flow_inference_batched_streaming(loaded, toks, prompts, xvec, [False, True])
    sb = fcv.flow_inference_batched_streaming(fe, toks, prompts, xvec, [False, True])
    assert all(torch.equal(x, y) for x, y in zip(sa, sb))
