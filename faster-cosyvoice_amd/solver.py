"""Packed CFG Euler solver over ``DiTEstimator`` (flashinfer_flow.py:16-74).

``solve_euler_packed`` keeps the sample packed and fp32 across steps and runs the whole
n-step loop inside libfcvdit (``fcv_dit_solve``).  With ``use_graph`` the loop is replayed from
a hipGraph once the same capacity and buffers come back: a capacity's first solve runs eagerly
and its second captures the graph, since a capture costs more than one eager run.
``solve_euler_batched`` keeps the reference's padded signature for callers that hand it
``[B,80,T]`` tensors and a padding mask.

``use_graph`` left to the solver replays graphs for request groups of at least
``GRAPH_MIN_ROWS`` capacity rows and launches smaller ones eagerly (see there).

By default a solve plans its layout into a capacity bucket (``capacity_bucket``): the
kernels read the layout from device memory, so the graph captured for a bucket replays for
every later layout that fits it (a streaming step or a new batch composition), where an exact
plan's graph serves only that layout.  Results are bit-identical either way.
"""

from __future__ import annotations

from collections.abc import Sequence
from typing import Any

import torch

from . import _lib
from .estimator import DiTEstimator, _PackedRunner
from .streams import group_stream


def euler_schedule(n_steps: int) -> tuple[list[float], list[float]]:
    """Per-step (t, dt) of the cosine schedule with the reference's fp32 recurrence:
    ``time = span[0]; dt = span[1]-span[0]``; after each step ``time += dt`` and
    ``dt = span[step+1] - time`` (flashinfer_flow.py:34-43,71-73)."""
    span = torch.linspace(0, 1, n_steps + 1, dtype=torch.float32)
    span = 1 - torch.cos(span * 0.5 * torch.pi)
    time = span[0]
    dt = span[1] - span[0]
    ts, dts = [], []
    for step in range(1, n_steps + 1):
        ts.append(float(time))
        dts.append(float(dt))
        time = time + dt
        if step < n_steps:
            dt = span[step + 1] - time
    return ts, dts


def capacity_bucket(rows: int, n_docs: int) -> tuple[int, int]:
    """The capacity a packed CFG layout of ``rows`` rows in ``n_docs`` documents is planned
    into: rows rounded up to m * 2^e with m in 8..15 (at most 12.5 % above, at least 256),
    documents to a power of two.  Any two layouts in one bucket share its solve graphs."""
    cap = 256
    while cap < rows:
        cap *= 2
    # cap is the smallest power of two >= rows; the eighths of the power below refine it
    low = cap // 2
    for m in range(9, 17):
        if m * low // 8 >= rows:
            cap = max(256, m * low // 8)
            break
    docs = 2
    while docs < n_docs:
        docs *= 2
    return cap, docs


_BUFFER_SETS = 4  # solver buffer sets kept per runner: one per graph its handle can pool

# Smallest capacity (packed CFG rows of one request group) whose solve replays its hipGraph
# when the caller leaves ``use_graph`` to the solver.  An eager solve is one C-ABI call that
# enqueues the whole step from C++ faster than the GPU drains it, so a replay saves host time
# (0.10 against 0.44-0.49 ms per step for one request) but no device time; on one MI355X the
# replayed step was 2-4 % slower than the same kernels launched eagerly at 760-1100 rows and
# 1 % faster at config 3's request groups (~4.6k rows each).
GRAPH_MIN_ROWS = 4096


def _solver_buffers(runner: _PackedRunner, dims, rows_cap: int,
                    docs_cap: int) -> dict[str, torch.Tensor]:
    """Packed CFG input buffers for up to ``rows_cap`` rows in ``docs_cap`` documents.  A set
    per capacity is kept (the most recently used few), so the buffer pointers a captured graph
    was recorded with come back with its capacity and the graph can be replayed."""
    key = (rows_cap, docs_cap)
    sets = runner.__dict__.setdefault("_solver_bufs", {})
    bufs = sets.pop(key, None)
    if bufs is None:
        mel, dev = dims.mel_dim, runner.device
        z = lambda rows: torch.zeros(rows, mel, dtype=torch.float32, device=dev)
        bufs = {"x": z(rows_cap), "mu": z(rows_cap), "cond": z(rows_cap), "spks": z(docs_cap)}
        while len(sets) >= _BUFFER_SETS:
            sets.pop(next(iter(sets)))  # least recently used
    sets[key] = bufs  # most recently used last
    return bufs


def _schedule(estimator: DiTEstimator, n_steps: int, t_arr,
              stream: torch.cuda.Stream) -> tuple[torch.Tensor, torch.cuda.Event]:
    """The estimator's ``n_steps`` solve schedule: every step's modulation rows
    (``fcv_dit_schedule``), which every request group's solve reads.  They depend
    only on the weights, which are fixed once finalized, and on the cosine schedule's t values,
    which ``n_steps`` fixes, so they are computed once per step count, on ``stream``, and kept
    for the estimator's life (the buffer's pointer is part of the graphs captured over it).
    Returns the buffer and an event recorded after its computation, which a solve on another
    stream waits for."""
    cache = estimator.__dict__.setdefault("_schedules", {})
    hit = cache.get(n_steps)
    if hit is not None:
        return hit
    lib = _lib.load()
    nbytes = lib.fcv_dit_schedule_bytes(estimator._require(), n_steps)
    if nbytes == 0:
        raise ValueError("n_steps must be in [1, 64]")
    buf = torch.empty(nbytes, dtype=torch.uint8, device=estimator.device)
    if buf.data_ptr() % 256:
        raise RuntimeError("schedule buffer is not 256-byte aligned")
    with torch.cuda.stream(stream):
        buf.record_stream(stream)
        _lib.check(lib.fcv_dit_schedule(estimator._require(), t_arr, n_steps, buf.data_ptr(),
                                        buf.numel(), stream.cuda_stream))
        done = torch.cuda.Event()
        done.record(stream)
    cache[n_steps] = (buf, done)
    return buf, done


def _stream_for(runner: _PackedRunner) -> torch.cuda.Stream:
    # a non-default stream (hipGraph capture needs one), shared per group across the process
    return group_stream(runner.device, runner.group)


def default_concurrency(n_requests: int) -> int:
    """Request groups a solve runs by default: two (measured best on one MI355X: config 3
    -10 %, config 4 -7 %, config 5 even; three or four groups lose to smaller tiles)."""
    return 2 if n_requests >= 2 else 1


def request_groups(lengths: Sequence[int], n_groups: int) -> list[list[int]]:
    """Requests split into ``n_groups`` groups of about equal DiT cost, per request
    ``378 MFLOP x L + 90 kFLOP x L^2`` (dense rows, attention pairs), longest first onto the
    least loaded group.  Empty groups are dropped; each group lists its requests in order."""
    cost = lambda n: n * n + 4200 * n
    groups: list[list[int]] = [[] for _ in range(max(1, n_groups))]
    load = [0] * len(groups)
    for i in sorted(range(len(lengths)), key=lambda i: -cost(lengths[i])):
        g = load.index(min(load))
        groups[g].append(i)
        load[g] += cost(lengths[i])
    return [sorted(g) for g in groups if g]


def _solve_on(runner: _PackedRunner, dims, noise: torch.Tensor, mu: torch.Tensor,
              cond: torch.Tensor, spks: torch.Tensor, lengths: list[int], t_arr, dt_arr,
              n_steps: int, cfg_rate: float, streaming: bool, use_graph: bool | None,
              stream: torch.cuda.Stream, bucketed: bool,
              schedule: torch.Tensor) -> torch.Tensor:
    """One packed CFG solve on ``runner``, enqueued on ``stream`` (the caller orders it).  It
    reads its modulation rows from ``schedule`` (filled by ``fcv_dit_schedule``)."""
    rc, b = sum(lengths), len(lengths)
    capacity = capacity_bucket(2 * rc, 2 * b) if bucketed else None
    if use_graph is None:
        use_graph = (capacity or (2 * rc, 2 * b))[0] >= GRAPH_MIN_ROWS
    with torch.cuda.stream(stream):
        runner.plan(lengths + lengths, streaming, capacity)
        # persistent solver buffers: stable pointers let a captured graph be replayed; the
        # unconditional half [rc, 2 rc) of mu and cond and spks[b:2b] must read zero
        buf = _solver_buffers(runner, dims, *(capacity or (2 * rc, 2 * b)))
        buf["x"][:rc].copy_(noise)
        buf["x"][rc:2 * rc].copy_(noise)
        buf["mu"][:rc].copy_(mu)
        buf["mu"][rc:2 * rc].zero_()
        buf["cond"][:rc].copy_(cond)
        buf["cond"][rc:2 * rc].zero_()
        buf["spks"][:b].copy_(spks)
        buf["spks"][b:2 * b].zero_()
        _lib.check(_lib.load().fcv_dit_solve_scheduled(
            runner._require(), buf["x"].data_ptr(), buf["mu"].data_ptr(),
            buf["cond"].data_ptr(), buf["spks"].data_ptr(), dt_arr, n_steps,
            float(cfg_rate), schedule.data_ptr(), schedule.numel(), int(bool(use_graph)),
            stream.cuda_stream))
        return buf["x"][:rc].clone()


def solve_euler_packed(estimator: DiTEstimator, noise: torch.Tensor, mu: torch.Tensor,
                       cond: torch.Tensor, spks: torch.Tensor, lengths: Sequence[int],
                       n_steps: int = 10, cfg_rate: float = 0.7, streaming: bool = False,
                       use_graph: bool | None = None, concurrency: int | None = None,
                       bucketed: bool = True) -> torch.Tensor:
    """CFG Euler solve on packed request rows.

    noise, mu, cond: ``[Rc, 80]`` conditional rows of the B requests (doc-major);
    spks: ``[B, 80]``; lengths: the B request lengths.  The result ``[Rc, 80]`` fp32 is the
    sample after ``n_steps`` steps.

    The requests run as ``concurrency`` groups (default: 2 when there are at least 2
    requests), each a packed CFG batch ``[cond..., uncond...]`` (zero mu/cond/spks in the
    second half) on its own handle over the shared weights and its own stream, all launched
    before any is waited for.  One group's tail rounds and bandwidth-bound phases then overlap
    the other's matrix work.  The modulation rows of the schedule (one pass over the AdaLN
    weights) are computed on the caller's stream by the first
    solve of a step count and kept (``_schedule``); every group of every later solve reads
    them.  A document's result does not depend on what it is packed with, so the rows are
    bit-identical to one packed batch of all requests.

    ``bucketed`` plans each group into its capacity bucket (``capacity_bucket``), so a new
    layout in a bucket that has been captured replays its graph; False plans the exact layout.
    ``use_graph``: True replays graphs, False launches eagerly, None (default) replays them for
    groups of at least ``GRAPH_MIN_ROWS`` capacity rows.  Results are bit-identical either way.
    """
    lengths = [int(n) for n in lengths]
    rc = sum(lengths)
    dev = estimator.device
    f32 = lambda a: a.to(device=dev, dtype=torch.float32).contiguous()
    noise, mu, cond, spks = f32(noise), f32(mu), f32(cond), f32(spks)
    if noise.shape[0] != rc or mu.shape[0] != rc or cond.shape[0] != rc:
        raise ValueError(f"noise, mu and cond must hold {rc} rows")
    if spks.shape[0] != len(lengths):
        raise ValueError("spks must hold one row per request")
    n_groups = default_concurrency(len(lengths)) if concurrency is None else int(concurrency)
    if n_groups < 1:
        raise ValueError("concurrency must be >= 1")
    groups = request_groups(lengths, n_groups)
    ts, dts = euler_schedule(n_steps)
    t_arr = (_lib.c_float * n_steps)(*ts)
    dt_arr = (_lib.c_float * n_steps)(*dts)
    current = torch.cuda.current_stream(dev)
    runners = estimator.lanes(len(groups))
    schedule, scheduled = _schedule(estimator, n_steps, t_arr, current)
    if len(groups) == 1:
        stream = _stream_for(estimator)
        stream.wait_stream(current)
        stream.wait_event(scheduled)
        result = _solve_on(estimator, estimator.dims, noise, mu, cond, spks, lengths, t_arr,
                           dt_arr, n_steps, cfg_rate, streaming, use_graph, stream, bucketed,
                           schedule)
        current.wait_stream(stream)
        return result
    offs = [0]
    for n in lengths:
        offs.append(offs[-1] + n)
    # each group's rows, made on the caller's stream before the groups start
    group_rows = [torch.cat([torch.arange(offs[i], offs[i + 1]) for i in g]).to(dev)
                  for g in groups]
    parts = []
    streams = [_stream_for(r) for r in runners]
    for s in streams:  # every group waits for the caller's work only, not for each other
        s.wait_stream(current)
        s.wait_event(scheduled)
    for runner, stream, g, rows in zip(runners, streams, groups, group_rows):
        with torch.cuda.stream(stream):
            out = _solve_on(runner, estimator.dims, noise[rows], mu[rows], cond[rows], spks[g],
                            [lengths[i] for i in g], t_arr, dt_arr, n_steps, cfg_rate,
                            streaming, use_graph, stream, bucketed, schedule)
            rows.record_stream(stream)
        parts.append((rows, out))
    for s in streams:
        current.wait_stream(s)
    result = torch.empty(rc, noise.shape[1], dtype=torch.float32, device=dev)
    for rows, out in parts:
        out.record_stream(current)
        result[rows] = out
    return result


@torch.no_grad()
def solve_euler_batched(decoder: Any, noise: torch.Tensor, mu: torch.Tensor, mask: torch.Tensor,
                        speaker_embeddings: torch.Tensor, condition: torch.Tensor,
                        num_timesteps: int = 10, streaming: bool = False) -> torch.Tensor:
    """Drop-in for the reference's ``solve_euler_batched`` (flashinfer_flow.py:16-74).

    ``decoder.estimator`` must be a ``DiTEstimator``; ``decoder.inference_cfg_rate`` is the
    CFG rate.  Padded ``[B,80,T]`` in, ``[B,80,T]`` out; padded frames keep the noise, as in
    the reference (whose estimator returns zeros there).
    """
    estimator = decoder.estimator
    if not isinstance(estimator, DiTEstimator):
        raise TypeError("decoder.estimator must be a DiTEstimator")
    lengths = [int(v) for v in mask[:, 0].sum(-1).round().to(torch.int64).tolist()]
    batch, mel, _ = noise.shape
    pack = lambda a: torch.cat([a[b, :, :n].transpose(0, 1) for b, n in enumerate(lengths)])
    x = solve_euler_packed(estimator, pack(noise), pack(mu), pack(condition), speaker_embeddings,
                           lengths, num_timesteps, float(decoder.inference_cfg_rate), streaming)
    out = noise.to(device=x.device, dtype=torch.float32).clone()
    off = 0
    for b, n in enumerate(lengths):
        out[b, :, :n] = x[off:off + n].transpose(0, 1)
        off += n
    return out.to(noise.dtype)


def apply_mi355x(model: Any, device: torch.device | str = "cuda:0") -> DiTEstimator:
    """Install ``DiTEstimator`` as ``model.flow.decoder.estimator`` (apply_flashinfer,
    flashinfer_dit.py:951-988): same hyper-parameters as the estimator it replaces, its
    state dict loaded (RoPE buffers excepted), weights finalized."""
    old = model.flow.decoder.estimator
    depth = len(old.transformer_blocks)
    dim = old.proj_out.weight.shape[1]
    heads = old.transformer_blocks[0].attn.heads if hasattr(old.transformer_blocks[0].attn, "heads") else 16
    chunk = getattr(old, "static_chunk_size", 50)
    new = DiTEstimator(dim=dim, depth=depth, heads=heads, dim_head=dim // heads,
                       static_chunk_size=chunk, device=device)
    new.load_reference_state_dict(old.state_dict())
    new.finalize_weights()
    model.flow.decoder.estimator = new
    return new
