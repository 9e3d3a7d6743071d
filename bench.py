"""Benchmark: DiT mel-frames/s per Euler step on a packed CFG batch, one MI355X.

A step is one Euler step of the packed CFG batch: one 22-block DiT estimator forward over all
2B documents plus the CFG combine and Euler update.  The timed region is one hipGraph-captured
solve of exactly K steps (the graph is captured during warm-up), repeated R times; the value
is the median solve's (each solve bracketed by device synchronisations).  Prints one JSON line.

    python bench.py [--gpus 1] [--steps 10] [--warmup 10] [--replays 5] [--workload 3]
"""

from __future__ import annotations

import argparse
import importlib.util
import json
import os
import platform
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA (fp16 dense: the same 2.5 PFLOP/s)
PEAK_HBM_GBS = 8000.0
QKV_REPEAT = 8                # launches per probe event pair (amortises event overhead)


def _load_package():
    name = "faster_cosyvoice_amd"
    if name in sys.modules:
        return sys.modules[name]
    pkg_dir = REPO / "faster-cosyvoice_amd"
    spec = importlib.util.spec_from_file_location(name, pkg_dir / "__init__.py",
                                                  submodule_search_locations=[str(pkg_dir)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(fcv, sd, batch, budget_s: float = 12.0) -> dict:
    """fp32 torch-eager padded-SDPA DiT (the oracle restatement of the reference's torch path)
    on the host cores: one Euler step (DiT forward over a CFG stack padded to its longest
    request, then the CFG combine), on the first requests of the workload until the budget."""
    import torch
    if str(REPO) not in sys.path:
        sys.path.insert(0, str(REPO))
    from oracle import dit_oracle as O

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    order = list(range(batch.n_requests))
    frames = padded_rows = 0
    used = 0
    t_total = 0.0
    offs = [0]
    for n in batch.lengths:
        offs.append(offs[-1] + n)
    with torch.no_grad():
        # two requests at a time, padded to the longer one (the reference torch path pads)
        for i in range(0, len(order), 2):
            idx = order[i:i + 2]
            T = max(batch.lengths[j] for j in idx)
            B = len(idx)
            x = torch.zeros(2 * B, 80, T)
            mu = torch.zeros(2 * B, 80, T)
            cond = torch.zeros(2 * B, 80, T)
            mask = torch.zeros(2 * B, 1, T)
            spks = torch.zeros(2 * B, 80)
            for k, j in enumerate(idx):
                n, o = batch.lengths[j], offs[j]
                for half in (0, 1):
                    x[half * B + k, :, :n] = batch.noise[o:o + n].T
                    mask[half * B + k, 0, :n] = 1
                mu[k, :, :n] = batch.mu[o:o + n].T
                cond[k, :, :n] = batch.cond[o:o + n].T
                spks[k] = batch.spks[j]
            t = torch.full((2 * B,), 0.5)
            t0 = time.perf_counter()
            v = O.dit_forward(sd, x, mask, mu, t, spks, cond, streaming=batch.streaming)
            vc, vu = v[:B], v[B:]
            _ = x[:B] + 0.1 * (1.7 * vc - 0.7 * vu)
            t_total += time.perf_counter() - t0
            frames += 2 * sum(batch.lengths[j] for j in idx)
            padded_rows += 2 * B * T
            used += B
            if t_total >= budget_s:
                break
    return {
        "value": frames / t_total,
        "unit": "mel-frames/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"one Euler step (fp32 padded-SDPA DiT forward + CFG combine) on the CFG "
                   f"pairs of the first {used} of {batch.n_requests} requests, two requests per "
                   f"padded batch; {frames} valid frames, {padded_rows} padded rows, "
                   f"{t_total:.1f} s; padded rows/s {padded_rows / t_total:.1f}; "
                   f"host CPU: {cpu_model()}"),
    }


def measured_traffic(workload: str) -> dict | None:
    """HBM bytes per launch of the QKV GEMM from the committed rocprofv3 PMC summary
    (FETCH_SIZE and WRITE_SIZE passes scaled by a plain-copy calibration), when it was measured
    on this workload."""
    path = REPO / "profiles" / "qkv_gemm_ragged8_traffic.json"
    try:
        rec = json.loads(path.read_text())
    except (OSError, ValueError):
        return None
    return rec if rec.get("workload") == workload else None


PEAK_FP32_TFLOPS = 157.3      # MI355X dense fp32 matrix peak
FRONTEND_REPEAT = 20


def frontend_leg(fcv, batch, dev, cpu: bool) -> dict:
    """The Flow front-end (tokens -> packed mu rows) for the workload's requests: the
    three-kernel token-features call timed with HIP events on the launch stream over
    FRONTEND_REPEAT back-to-back calls on device-resident ids, plus the fp32 oracle on the
    host for the same requests (rank 0, one core budget of a few seconds)."""
    import torch
    dims = fcv.synthetic.FlowDims()
    sd = fcv.synthetic.random_flow_state_dict(dims, seed=0)
    fe = fcv.FlowFrontEnd(device=dev)
    fe.load_reference_state_dict(sd)
    fe.finalize_weights()
    g = torch.Generator().manual_seed(5)
    n_tok = [(n + dims.token_mel_ratio - 1) // dims.token_mel_ratio for n in batch.lengths]
    token_list = [torch.randint(0, dims.vocab, (n,), generator=g).tolist() for n in n_tok]
    tokens = torch.tensor([v for t in token_list for v in t], dtype=torch.int32, device=dev)
    out = torch.empty(dims.token_mel_ratio * sum(n_tok), dims.feat, device=dev)
    for _ in range(3):
        fe.token_features_device(tokens, n_tok, out=out)
    stream = torch.cuda.current_stream(dev)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(FRONTEND_REPEAT):
        fe.token_features_device(tokens, n_tok, out=out)
    stop.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / FRONTEND_REPEAT
    tokens_total = sum(n_tok)
    flop_per_token = 2 * (dims.channels * (dims.lookahead + 1) * dims.feat
                          + dims.feat * 3 * dims.channels)
    tflops = flop_per_token * tokens_total / (ms * 1e-3) / 1e12
    res = {
        "what": "token embedding + PreLookaheadLayer + repeat to Mel rows (3 kernels, fp32)",
        "requests": len(n_tok), "tokens": tokens_total,
        "ms_per_call": round(ms, 4),
        "tokens_per_s": round(tokens_total / (ms * 1e-3), 1),
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_FP32_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_FP32_TFLOPS, 4),
                     "flop_per_token": flop_per_token,
                     "timing": f"HIP events around {FRONTEND_REPEAT} back-to-back calls"},
    }
    if cpu:
        from oracle import frontend_oracle as FO
        torch.set_num_threads(1)
        empty = [torch.zeros(1, 0, dims.feat)] * len(n_tok)
        t0 = time.perf_counter()
        FO.flow_inputs(sd, token_list, empty, torch.ones(len(n_tok), dims.spk_dim))
        cpu_s = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": round(tokens_total / cpu_s, 1), "unit": "tokens/s",
                               "cores": 1, "kind": "port",
                               "sample": "the same requests through the fp32 oracle front-end "
                                         "(padded batch, torch CPU conv1d)"}
    return res


HIFT_REPEAT = 3


def hift_leg(fcv, batch, dev, cpu: bool) -> dict:
    """The HiFT vocoder on the generated Mel of the workload's requests (request length minus
    its prompt), one ``inference_batched`` call (two concurrent packed request groups): HIP
    events on the caller's stream around HIFT_REPEAT calls; plus the fp32/fp64 oracle on the
    host for a bounded sample."""
    import torch
    dims = fcv.synthetic.HiFTDims()
    gen = [n - p for n, p in zip(batch.lengths, batch.prompt_lengths)]
    sd = fcv.synthetic.random_hift_state_dict(dims, seed=0)
    buf = fcv.synthetic.random_hift_buffers(dims, max_samples=dims.upsample_scale * max(gen),
                                            seed=1)
    voc = fcv.HiFTVocoder(dims, device=dev, buffers=buf)
    voc.load_reference_state_dict(sd)
    voc.finalize_weights()
    g = torch.Generator().manual_seed(6)
    mels = [torch.randn(80, n, generator=g).to(dev) for n in gen]
    voc.inference_batched(mels)
    voc.inference_batched(mels)  # each group's capacity graph is captured here
    stream = torch.cuda.current_stream(dev)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(graph: bool, ms_in=mels, fin=None, repeat=HIFT_REPEAT) -> float:
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(repeat):
            voc.inference_batched(ms_in, fin, graph=graph)
        stop.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / repeat

    ms = timed(True)
    ms_eager = timed(False)
    # one streaming chunk: 60 new Mel frames after 8 frames of right context, not final
    chunk = [torch.randn(80, 68, generator=g).to(dev)]
    voc.inference_batched(chunk, [False])
    voc.inference_batched(chunk, [False])
    # replay and eager alternate, five rounds of 20 calls each, medians: back-to-back blocks
    # of one and then the other picked up host-side drift (other legs' CPU work) as a
    # replay/eager difference
    rounds = [(timed(True, chunk, [False], 20), timed(False, chunk, [False], 20))
              for _ in range(5)]
    chunk_ms = sorted(r[0] for r in rounds)[2]
    chunk_eager = sorted(r[1] for r in rounds)[2]
    frames = sum(gen)
    audio_s = frames * dims.upsample_scale / dims.sampling_rate
    macs = fcv.synthetic.hift_macs_per_frame(dims)
    flop = 2.0 * frames * sum(v for k, v in macs.items() if k != "f0_fp64")
    tflops = flop / (ms * 1e-3) / 1e12
    res = {
        "what": "HiFT vocoder, Mel -> 24 kHz waveform, the requests as two concurrent packed "
                "request groups (fp32, F0 predictor fp64)",
        "requests": len(gen), "mel_frames": frames, "audio_seconds": round(audio_s, 2),
        "ms_per_call": round(ms, 3),
        "eager_ms_per_call": round(ms_eager, 3),
        "stream_chunk": {"what": "one non-final request of 68 Mel frames (60 new + 8 right "
                                 "context), median of 5 alternating rounds of 20 replayed and "
                                 "20 eager calls", "ms_per_call": round(chunk_ms, 4),
                         "eager_ms_per_call": round(chunk_eager, 4)},
        "audio_seconds_per_second": round(audio_s / (ms * 1e-3), 1),
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_FP32_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_FP32_TFLOPS, 4),
                     "flop_per_frame": 2 * sum(v for k, v in macs.items() if k != "f0_fp64"),
                     "timing": f"HIP events around {HIFT_REPEAT} back-to-back calls replayed from "
                               "the groups' capacity graphs; achieved counts the fp32 "
                               "convolutions of the whole call"},
    }
    if cpu:
        from oracle import hift_oracle as HO
        threads = len(os.sched_getaffinity(0))
        torch.set_num_threads(threads)
        folded = HO.fold_weight_norm(sd)
        n = min(gen[0], 200)
        mel = mels[0][:, :n].cpu()[None]
        t0 = time.perf_counter()
        HO.inference(folded, mel, buf, dims, True)
        cpu_s = time.perf_counter() - t0
        res["cpu_baseline"] = {
            "value": round(n * dims.upsample_scale / dims.sampling_rate / cpu_s, 2),
            "unit": "audio seconds per second", "cores": threads, "kind": "port",
            "sample": f"the first request's first {n} Mel frames through the oracle vocoder "
                      "(torch CPU conv1d, fp32; F0 in fp64)"}
    return res


def token2wav_leg(fcv, est, batch, dev) -> dict:
    """The whole Token2Wav pass for the workload's requests, tokens to waveform: front-end,
    the packed 10-step CFG solve on the 22-block estimator, HiFT on the generated Mel in one
    packed call (flashinfer_flow.py:118-184 then token2wav.py:128-131).  Wall time with a
    device synchronisation on both sides, two calls after one untimed."""
    import torch
    fdims = fcv.synthetic.FlowDims()
    fe = fcv.FlowFrontEnd(device=dev)
    fe.load_reference_state_dict(fcv.synthetic.random_flow_state_dict(fdims, seed=0))
    fe.finalize_weights()
    fe.decoder = fcv.CFMDecoder(est)
    hdims = fcv.synthetic.HiFTDims()
    n_tok = [(n + 1) // 2 for n in batch.lengths]
    p_tok = [p // 2 for p in batch.prompt_lengths]
    voc = fcv.HiFTVocoder(hdims, device=dev, buffers=fcv.synthetic.random_hift_buffers(
        hdims, max_samples=hdims.upsample_scale * 2 * max(n_tok), seed=1))
    voc.load_reference_state_dict(fcv.synthetic.random_hift_state_dict(hdims, seed=0))
    voc.finalize_weights()
    g = torch.Generator().manual_seed(7)
    tokens = [torch.randint(0, fdims.vocab, (n,), generator=g).tolist() for n in n_tok]
    prompts = [torch.randn(1, 2 * p, 80, generator=g) for p in p_tok]
    xvec = torch.randn(len(n_tok), 192, generator=g).to(dev)

    def run():
        mels = fcv.flow_inference_batched(fe, tokens, prompts, xvec)
        return voc.inference_batched(mels)

    run()
    times = []
    for _ in range(2):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        wavs = run()
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    sec = min(times)
    audio = sum(w.shape[1] for w in wavs) / hdims.sampling_rate
    return {"what": "tokens -> 24 kHz waveform: front-end, 10-step CFG solve (22 blocks, "
                    "hipGraph), HiFT, all requests packed",
            "requests": len(n_tok), "tokens": sum(n_tok), "audio_seconds": round(audio, 2),
            "ms_per_batch": round(sec * 1e3, 2),
            "audio_seconds_per_second": round(audio / sec, 1),
            "timing": "wall clock with torch.cuda.synchronize() on both sides, best of 2"}


def chunk_plans(prompt_tokens: int, total: int, chunk: int = 15, lookahead: int = 3,
                scale: int = 2) -> list[tuple[int, int, bool]]:
    """(prefix_len, token_offset, finalize) of every chunk of a session whose tokens all arrive
    before token2wav asks for them, by the reference's planner rules (streaming/chunker.py:
    20-56): the first hop is ``chunk`` tokens plus the pad that aligns the prompt to a multiple
    of ``chunk``; each chunk also reads ``lookahead`` tokens it does not consume; the hop then
    grows by ``scale`` up to four times ``chunk``; what is left at the end is one final chunk."""
    pad = (-prompt_tokens) % chunk if prompt_tokens > 0 else 0
    hop, done, plans = chunk, 0, []
    while True:
        this = hop + (pad if done == 0 else 0)
        if total - done < this + lookahead:
            break
        plans.append((done + this + lookahead, done, False))
        done += this
        hop = min(4 * chunk, max(chunk, hop * scale))
    if total > done:
        plans.append((total, done, True))
    return plans


def stream_leg(fcv, est, batch, dev) -> dict:
    """Packed streaming steps (token2wav.py:203-226 with the packed vocoder): the workload's
    requests as concurrent sessions, every session's next chunk in one
    ``StreamingFlow.stream_step_batched`` call (front-end over the full token prefix, the
    chunk-causal 10-step CFG solve from the fixed noise prefix on the 22-block estimator, one
    packed HiFT call over the sessions' Mel caches), until every session has emitted its final
    chunk.  Wall time of each step between device synchronisations, on a second pass over fresh
    sessions (the first, untimed, captures the capacity graphs); plus one session's first chunk
    alone, the token2wav share of a time-to-first-packet at concurrency 1."""
    import copy
    from types import SimpleNamespace

    import torch
    fdims = fcv.synthetic.FlowDims()
    fe = fcv.FlowFrontEnd(device=dev)
    fe.load_reference_state_dict(fcv.synthetic.random_flow_state_dict(fdims, seed=0))
    fe.finalize_weights()
    fe.decoder = fcv.CFMDecoder(est)
    hdims = fcv.synthetic.HiFTDims()
    p_tok = [p // 2 for p in batch.prompt_lengths]
    n_tok = [max(1, (n - p) // 2) for n, p in zip(batch.lengths, batch.prompt_lengths)]
    voc = fcv.HiFTVocoder(hdims, device=dev, buffers=fcv.synthetic.random_hift_buffers(
        hdims, max_samples=hdims.upsample_scale * 2 * max(n_tok), seed=1))
    voc.load_reference_state_dict(fcv.synthetic.random_hift_state_dict(hdims, seed=0))
    voc.finalize_weights()
    sf = fcv.StreamingFlow(fe, vocoder=voc.inference)
    g = torch.Generator().manual_seed(8)
    sessions = []
    for p, n in zip(p_tok, n_tok):
        cond = SimpleNamespace(
            prompt_tokens_flow=torch.randint(0, fdims.vocab, (p,), generator=g).tolist(),
            prompt_feat=torch.randn(1, 2 * p, 80, generator=g),
            spk_embedding=torch.randn(192, generator=g))
        sessions.append(SimpleNamespace(
            cond=cond, tokens=torch.randint(0, fdims.vocab, (n,), generator=g).tolist(),
            mel_cache=None, speech_offset=0, chunk_index=0))
    plans = [[SimpleNamespace(prefix_len=a, token_offset=b, finalize=c)
              for a, b, c in chunk_plans(p, n)] for p, n in zip(p_tok, n_tok)]

    def run(timed: bool):
        live = copy.deepcopy(sessions)
        step_ms, samples = [], 0
        for k in range(max(len(pl) for pl in plans)):
            idx = [i for i, pl in enumerate(plans) if k < len(pl)]
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            pcm = sf.stream_step_batched([live[i] for i in idx], [plans[i][k] for i in idx])
            torch.cuda.synchronize()
            step_ms.append((time.perf_counter() - t0) * 1e3)
            samples += sum(x.shape[-1] for x in pcm)
        return step_ms, samples

    run(False)
    step_ms, samples = run(True)

    def first_alone() -> float:
        s = copy.deepcopy(sessions[0])
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        sf.stream_step(s, plans[0][0])
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3

    first_alone()
    alone = sorted(first_alone() for _ in range(3))[1]
    total_ms = sum(step_ms)
    audio = samples / hdims.sampling_rate
    return {"what": "packed streaming steps, tokens -> PCM: front-end over each session's full "
                    "token prefix, chunk-causal 10-step CFG solve (22 blocks) from the fixed "
                    "noise prefix, one packed HiFT call over the sessions' Mel caches",
            "sessions": len(sessions), "prompt_tokens": p_tok, "tokens": n_tok,
            "chunk_plan": "15-token first hop plus the prompt-alignment pad, 3 lookahead "
                          "tokens, hop doubling to 60, final remainder "
                          "(streaming/chunker.py:20-56); all tokens available up front",
            "steps": len(step_ms), "step_ms": [round(v, 2) for v in step_ms],
            "ms_total": round(total_ms, 2), "audio_seconds": round(audio, 2),
            "audio_seconds_per_second": round(audio / (total_ms * 1e-3), 1),
            "first_chunk_ms": {"packed_sessions": round(step_ms[0], 2),
                               "one_session_alone": round(alone, 2)},
            "timing": "wall clock with torch.cuda.synchronize() around each step; the second "
                      "pass over fresh copies of the sessions (the first captures graphs); "
                      "one session alone: median of 3 after one untimed call"}


def _group_caps(fcv, b) -> tuple:
    """Capacity bucket of each request group the solver makes of batch `b`."""
    groups = fcv.solver.request_groups(b.lengths, fcv.solver.default_concurrency(b.n_requests))
    return tuple(fcv.solver.capacity_bucket(2 * sum(b.lengths[i] for i in g), 2 * len(g))
                 for g in groups)


def _fresh_layouts(fcv, est, base, variants, K: int) -> dict:
    """Solve `base` twice (each request group's capacity bucket gets its graph on the second),
    then time each variant (a layout never seen before, in the same buckets) replayed from
    those graphs, solved eagerly in the same buckets (the replay's kernels and grids, launched
    one by one: the graph's own effect) and solved eagerly on exact plans."""
    import torch

    def solve(b, graph, bucketed):
        return fcv.solve_euler_packed(est, b.noise, b.mu, b.cond, b.spks, b.lengths, n_steps=K,
                                      streaming=b.streaming, use_graph=graph, bucketed=bucketed)

    lanes = est.lanes(len(_group_caps(fcv, base)))
    captures = lambda: sum(r.graph_stats()[1] for r in lanes)
    solve(base, True, True)
    solve(base, True, True)  # the buckets' graphs are captured here
    captured = captures()

    def timed(b, graph, bucketed):
        # (wall ms per step, ms per step the calling thread spent inside the solve call)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        solve(b, graph, bucketed)
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / K, (t1 - t0) * 1e3 / K

    replay, eager_bucketed, eager = [], [], []
    for v in variants:  # interleaved, so drift between the three falls on all of them
        replay.append(timed(v, True, True))
        eager_bucketed.append(timed(v, False, True))
        eager.append(timed(v, False, False))
    new_captures = captures() - captured
    med = lambda xs, i=0: round(sorted(x[i] for x in xs)[len(xs) // 2], 4)
    return {"request_groups": len(lanes), "capacities": [list(c) for c in _group_caps(fcv, base)],
            "layouts": len(variants), "rows": [v.rows for v in variants],
            "captures_during_replays": new_captures,
            "replay_ms_per_step": med(replay),
            "eager_bucketed_ms_per_step": med(eager_bucketed),
            "eager_ms_per_step": med(eager),
            "host_ms_per_step": {"replay": med(replay, 1), "eager_bucketed": med(eager_bucketed, 1),
                                 "eager": med(eager, 1)}}


def fresh_layout_leg(fcv, est, batch, K: int, n_layouts: int = 4) -> dict:
    """K-step solves of layouts the solver has never seen, replayed from the graphs captured
    for their capacity buckets on another layout, against eager exact plans of the same layouts
    (wall clock between device synchronisations, median over the layouts):
    (a) the workload with every request length moved by a seeded -20..20 frames, kept when each
    request group stays in its bucket (the default two concurrent groups);
    (b) one request (a single streaming session for the chunk-causal workload) of a new length
    each solve, all in one bucket."""
    import numpy as np
    out = {"what": "graph replay of new layouts in captured capacity buckets vs eager exact "
                   "plans", "timing": "median over the layouts; wall clock with "
                   "torch.cuda.synchronize() on both sides; host_ms_per_step: time the calling "
                   "thread spends inside the solve call (enqueue, before the synchronize)"}
    rng = np.random.Generator(np.random.PCG64(7))
    variants = []
    for _ in range(200):
        lengths = [max(8, n + int(d)) for n, d in zip(batch.lengths,
                                                      rng.integers(-20, 21, batch.n_requests))]
        prompts = [min(p, n - 1) for p, n in zip(batch.prompt_lengths, lengths)]
        v = fcv.synthetic.make_batch("fresh", lengths, prompts, seed=int(rng.integers(1 << 30)),
                                     streaming=batch.streaming)
        if _group_caps(fcv, v) == _group_caps(fcv, batch):
            variants.append(v)
        if len(variants) == n_layouts:
            break
    if variants:
        out["workload"] = _fresh_layouts(fcv, est, batch, variants, K)
    # single request: 60 new frames after prompts of 295..320 frames (all in one bucket)
    single = [fcv.synthetic.make_batch("single", [p + 60], [p], seed=100 + p,
                                       streaming=batch.streaming)
              for p in (300, 295, 305, 312, 320)]
    assert all(_group_caps(fcv, v) == _group_caps(fcv, single[0]) for v in single)
    out["single_request"] = _fresh_layouts(fcv, est, single[0], single[1:], K)
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--replays", type=int, default=5,
                    help="timed K-step solves; value is the median one's")
    ap.add_argument("--groups", type=int, default=0,
                    help="request groups the solve runs concurrently (0: the solver's default)")
    ap.add_argument("--workload", type=int, default=3, choices=[2, 3, 4, 5])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-breakdown", action="store_true")
    ap.add_argument("--no-frontend", action="store_true", help="skip the flow front-end leg")
    ap.add_argument("--no-hift", action="store_true", help="skip the HiFT vocoder leg")
    ap.add_argument("--no-token2wav", action="store_true",
                    help="skip the end-to-end tokens -> waveform leg")
    ap.add_argument("--no-stream", action="store_true",
                    help="skip the packed streaming-step leg (tokens -> PCM chunks)")
    ap.add_argument("--eager", action="store_true", help="launch kernels one by one (no hipGraph)")
    ap.add_argument("--no-fresh-layouts", action="store_true",
                    help="skip the leg that solves new layouts through the bucket's graph")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 5 device-to-device copies of MIB MiB (counter calibration)")
    args = ap.parse_args()
    if args.copy_calibration:
        import torch
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_mib": args.copy_calibration, "launches": 5}))
        return 0
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the estimator runs on a single MI355X "
              "(documents would shard across GPUs without any collective)",
              file=sys.stderr)
        return 2
    if not 1 <= args.steps <= 64:
        print("--steps must be in [1, 64]", file=sys.stderr)
        return 2

    import torch
    fcv = _load_package()
    from faster_cosyvoice_amd import _lib

    dev = torch.device("cuda:0")
    batch = fcv.synthetic.workload(args.workload)
    log(f"[bench] workload {batch.name}: {batch.n_requests} requests, {len(batch.doc_lengths)} "
        f"packed docs, {batch.rows} rows")
    log("[bench] drawing 22-layer weights (seed 0)")
    sd = fcv.synthetic.random_state_dict(fcv.synthetic.DiTDims(), seed=0)
    est = fcv.DiTEstimator(depth=22, device=dev)
    est.load_reference_state_dict(sd)
    est.finalize_weights()
    lib = _lib.load()
    handle = est._require()

    K = args.steps

    def solve(graph: bool, concurrency: int | None = args.groups or None):
        return fcv.solve_euler_packed(est, batch.noise, batch.mu, batch.cond, batch.spks,
                                      batch.lengths, n_steps=K, streaming=batch.streaming,
                                      use_graph=graph, concurrency=concurrency)

    def probed_eager(stage: int, repeat: int = 1) -> tuple[list[float], float]:
        """One eager K-step solve with HIP events around `stage` (in block 1, whose launches
        every later block repeats; the LN-modulate pass in block 0) every step; with
        repeat > 1 the probed launch runs `repeat` times back to back inside the pair and the
        library reports the per-launch time."""
        _lib.check(lib.fcv_dit_probe_arm(handle, stage, K, repeat))
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        solve(False, concurrency=1)  # one packed batch on the probed handle: kernels alone
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        buf = (_lib.c_float * K)()
        n = _lib.c_int32()
        _lib.check(lib.fcv_dit_probe_read(handle, buf, K, n))
        _lib.check(lib.fcv_dit_probe_arm(handle, stage, 0, 1))
        return [buf[i] for i in range(min(n.value, K))], wall

    log("[bench] warm-up")
    for _ in range(max(1, -(-args.warmup // K))):
        solve(False)
    torch.cuda.synchronize()

    # timed region 1: the dominant kernel (QKV GEMM), HIP events on its stream, eager launches;
    # each pair brackets QKV_REPEAT back-to-back launches of block 1's QKV GEMM (the launch
    # every later block repeats)
    log(f"[bench] timing {K} steps eagerly with events around the QKV GEMM")
    qkv_ms, probed_wall = probed_eager(0, QKV_REPEAT)
    qkv_avg = sum(qkv_ms) / len(qkv_ms)

    # an unprobed eager solve with the same request groups as the timed replays (kernels
    # launched one by one, no events), for the eager-versus-graph comparison
    log(f"[bench] timing 3 x {K} steps eagerly (same request groups, no probe)")
    eager_s = []
    for _ in range(3):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        solve(False)
        torch.cuda.synchronize()
        eager_s.append(time.perf_counter() - t0)
    eager_wall = sorted(eager_s)[1]

    # timed region 2: the metric, K steps replayed from one hipGraph (captured before timing)
    if not args.eager:
        # a layout is captured on its second graph solve (the probes above re-planned the
        # first handle), so two untimed calls leave every group's graph captured
        solve(True)
        solve(True)
        torch.cuda.synchronize()
    log(f"[bench] timing {args.replays} x {K} steps" + ("" if args.eager else " (hipGraph replay)"))
    replay_s = []
    for _ in range(max(1, args.replays)):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        solve(not args.eager)
        torch.cuda.synchronize()
        replay_s.append(time.perf_counter() - t0)
    elapsed = sorted(replay_s)[len(replay_s) // 2]

    rows = batch.rows
    flops = fcv.synthetic.flops_per_forward(batch.doc_lengths, batch.streaming)
    ms_per_step = elapsed * 1e3 / K
    value = rows * K / elapsed
    qkv_flops = 2.0 * rows * 1024 * 3072
    achieved = qkv_flops / (qkv_avg * 1e-3) / 1e12
    traffic = measured_traffic(batch.name)
    mfma_util = flops["total"] / (ms_per_step * 1e-3) / (PEAK_BF16_TFLOPS * 1e12)

    breakdown = {}
    if not args.no_breakdown:
        log("[bench] per-stage breakdown (eager, events around each stage in block 1)")
        for stage, name in enumerate(_lib.STAGES):
            accumulates = name in ("out_proj", "ff2", "euler", "forward")
            vals, _ = probed_eager(stage, 1 if accumulates else QKV_REPEAT)
            if vals:
                breakdown[name] = round(sum(vals) / len(vals), 4)

    fresh = None
    if not args.no_fresh_layouts:
        log("[bench] new layouts through the capacity bucket's graph")
        fresh = fresh_layout_leg(fcv, est, batch, K)

    frontend = None
    if not args.no_frontend:
        log("[bench] flow front-end (tokens -> packed mu rows)")
        frontend = frontend_leg(fcv, batch, dev, cpu=not args.no_cpu_baseline)

    hift = None
    if not args.no_hift:
        log("[bench] HiFT vocoder (generated Mel -> waveform)")
        hift = hift_leg(fcv, batch, dev, cpu=not args.no_cpu_baseline)

    t2w = None
    if not args.no_token2wav:
        log("[bench] Token2Wav pass (tokens -> waveform)")
        t2w = token2wav_leg(fcv, est, batch, dev)

    stream_res = None
    if not args.no_stream:
        log("[bench] packed streaming steps (tokens -> PCM chunks)")
        stream_res = stream_leg(fcv, est, batch, dev)

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (fp32 oracle, padded SDPA)")
        cpu = cpu_baseline(fcv, sd, batch)

    out = {
        "metric": "DiT mel-frames/sec per Euler step (packed CFG batch); MFMA util % of bf16 peak",
        "value": round(value, 1),
        "unit": "mel-frames/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded N(0,1) inputs, N(0,0.02) random-init weights)",
        "config": {
            "workload": batch.name,
            "description": {2: "1 request x 550 frames, CFG pair, 22 blocks",
                            3: "8 requests, lengths U[100,1500], CFG -> 16 packed docs, full attention, cosine-schedule Euler",
                            4: "32 streams, prefix U(150,400) + hop {30,60,120}, CFG -> 64 docs, chunk-causal (50)",
                            5: "64 requests, LogNormal(800,0.6) clipped [64,3000], CFG -> 128 docs, full attention"}[args.workload],
            "requests": batch.n_requests,
            "packed_docs": len(batch.doc_lengths),
            "rows_per_step": rows,
            "depth": 22, "dim": 1024, "heads": 16,
            "graph": "none (eager launches)" if args.eager else "hipGraph of the K-step solve",
            "request_groups": len(fcv.solver.request_groups(
                batch.lengths, args.groups or fcv.solver.default_concurrency(batch.n_requests))),
            "concurrency": ("requests split into cost-balanced groups, each a packed CFG batch "
                            "on its own handle and stream, all launched before any is waited "
                            "for; rows bit-identical to one packed batch"),
        },
        # rows count both CFG halves; a request's frames appear once per half
        "request_frames_per_s": round(value / 2, 1),
        "mfma_util_pct": round(100 * mfma_util, 2),
        "tflops_per_step": round(flops["total"] / 1e12, 4),
        "roofline": {
            "kernel": ("qkv_gemm (bias + RoPE + head-major q/k and transposed V scatter), "
                       "block 1, every step"),
            "timing": (f"HIP events (no system fence) on the launch stream around {QKV_REPEAT} "
                       "back-to-back launches of block 1's QKV GEMM, every step of an eager "
                       "K-step solve"),
            "bound": "mfma",
            "achieved": round(achieved, 1),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": traffic["bytes_per_launch"] if traffic else None,
            "traffic_source": (f"rocprofv3 --pmc FETCH_SIZE x{traffic['fetch_scale']} + "
                               f"WRITE_SIZE x{traffic['write_scale']} per dispatch "
                               f"({traffic['source']})") if traffic else None,
            "avg_ms": round(qkv_avg, 5),
            "flop_per_launch": qkv_flops,
        },
        "cpu_baseline": cpu,
        "stage_ms": breakdown,
        "fresh_layouts": fresh,
        "frontend": frontend,
        "hift": hift,
        "token2wav": t2w,
        "stream": stream_res,
        "eager_ms_per_step": round(eager_wall * 1e3 / K, 4),
        "eager_timing": (f"median of 3 eager {K}-step solves with the replays' request groups, "
                         "each between torch.cuda.synchronize() calls"),
        "probed_solve_ms_per_step": round(probed_wall * 1e3 / K, 4),
        "probed_solve_timing": (f"the roofline probe's eager solve: one request group, HIP "
                                f"events every step, block 1's QKV GEMM launched {QKV_REPEAT} "
                                "times per step"),
        "replay_ms_per_step": [round(v * 1e3 / K, 4) for v in replay_s],
        "timing": (f"median of {len(replay_s)} timed {K}-step solves, each between "
                   "torch.cuda.synchronize() calls"),
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
