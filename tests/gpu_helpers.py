"""Helpers shared by the GPU parity tests (estimator construction, oracle calls, metrics)."""

from __future__ import annotations

import sys

import torch

from oracle import dit_oracle as O


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.double().cpu(), b.double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def say(*args) -> None:
    print(*args, flush=True)
    sys.stdout.flush()


def f16_weights(sd: dict) -> dict:
    """The oracle's view of the weights the GPU path stores in fp16 (biases stay fp32)."""
    return {k: (v.to(torch.float16).float() if k.endswith("weight") else v) for k, v in sd.items()}


def make_estimator(fcv, sd: dict, depth: int, **kw):
    est = fcv.DiTEstimator(depth=depth, device="cuda:0", **kw)
    est.load_reference_state_dict(sd)
    est.finalize_weights()
    return est


def oracle_packed(sd, x, mu, cond, spks, t, lengths, streaming=False, chunk=50):
    return O.dit_forward_packed(sd, x.cpu(), mu.cpu(), cond.cpu(), spks.cpu(), t.cpu(), lengths,
                                streaming=streaming, chunk_size=chunk)


def random_packed(lengths, seed=0, t=None):
    g = torch.Generator().manual_seed(seed)
    R, N = sum(lengths), len(lengths)
    x, mu, cond = (torch.randn(R, 80, generator=g) for _ in range(3))
    spks = torch.randn(N, 80, generator=g)
    tt = torch.rand(N, generator=g) if t is None else torch.full((N,), float(t))
    return x, mu, cond, spks, tt
