"""fcv_flow_token_features_noalloc (include/fcv_flow.h): the token-features call with the
library's own device scratch instead of a caller workspace.  Two calls in a row, the second
smaller, each give bit for bit what fcv_flow_token_features gives with a caller workspace; a
call past the scratch limit is refused with a clear message before anything is launched."""

from __future__ import annotations

import pytest
import torch

from tests.gpu_helpers import say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _front_end(fcv):
    dims = fcv.synthetic.FlowDims()
    fe = fcv.FlowFrontEnd(device="cuda:0")
    fe.load_reference_state_dict(fcv.synthetic.random_flow_state_dict(dims, seed=81))
    fe.finalize_weights()
    return fe


def _noalloc(fcv, fe, tokens, lengths, finalize, out):
    lib = fcv._lib.load()
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    return lib.fcv_flow_token_features_noalloc(
        fe.dims, fe._require(), tokens.data_ptr(), (fcv._lib.c_int32 * len(cu))(*cu),
        (fcv._lib.c_int32 * len(finalize))(*[int(f) for f in finalize]), len(lengths),
        out.data_ptr(), torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("case", ["large_then_small"])
def test_noalloc_matches_workspace_call(fcv, case):
    fe = _front_end(fcv)
    g = torch.Generator().manual_seed(82)
    calls = [([700, 1, 455, 1200, 33, 1300], [True, True, False, True, False, True]),
             ([90, 12], [False, True])]
    for lengths, fin in calls:
        ids = torch.randint(-3, 6561, (sum(lengths),), generator=g, dtype=torch.int32)
        tokens = ids.to("cuda:0")
        say(f"[noalloc] {len(lengths)} documents, {sum(lengths)} tokens")
        want, _ = fe.token_features_device(tokens, lengths, fin)
        got = torch.full_like(want, float("nan"))
        fcv._lib.check(_noalloc(fcv, fe, tokens, lengths, fin, got))
        torch.cuda.synchronize()
        assert torch.equal(got, want)


def test_noalloc_refuses_calls_past_its_scratch(fcv):
    fe = _front_end(fcv)
    n = 5042  # one output token more than 32 MiB of scratch holds at these dims
    tokens = torch.zeros(n, dtype=torch.int32, device="cuda:0")
    out = torch.empty(2 * n, 80, device="cuda:0")
    rc = _noalloc(fcv, fe, tokens, [n], [True], out)
    assert rc == fcv._lib.FCV_ERR_INVALID
    msg = fcv._lib.load().fcv_last_error().decode()
    assert "no-allocation entry point holds 33554432" in msg and "at most 5041" in msg
    ok_tokens = torch.zeros(5041, dtype=torch.int32, device="cuda:0")
    fcv._lib.check(_noalloc(fcv, fe, ok_tokens, [5041], [True], out))
    torch.cuda.synchronize()
    assert torch.isfinite(out[:2 * 5041]).all()
