"""``HiFTVocoder``: the MI355X drop-in for the reference's ``CausalHiFTGenerator`` (Mel -> 24 kHz
waveform, hifigan/generator.py:578-735), compute in libfcvdit.so (include/fcv_hift.h).

Holds the reference's parameters under their ``hift.pt`` names (``conv_pre.parametrizations.
weight.original0`` ...; a ``generator.`` prefix is accepted, token2wav.py:71-74) and the causal
source's fixed random buffers.  ``finalize_weights`` folds weight norm, packs every conv weight
as [ceil64(cout)][k][ceil16(cin)], and keeps the F0 predictor in fp64 as the reference does
(generator.py:722).  ``inference(speech_feat, finalize)`` has the reference's signature;
``inference_batched`` vocodes several requests of different lengths in one packed call.
"""

from __future__ import annotations

from collections.abc import Sequence

import numpy as np
import torch
from scipy.signal import get_window

from . import _lib
from .streams import group_stream
from .synthetic import HiFTDims, hift_state_dict_shapes, random_hift_buffers

_G = ".parametrizations.weight.original0"
_V = ".parametrizations.weight.original1"


def _ceil(v: int, m: int) -> int:
    return (v + m - 1) // m * m


# Smallest capacity (Mel frames of one packed call) whose call replays its captured graph when
# the caller leaves ``graph`` to the vocoder.  The eager call is one C-ABI call that enqueues the
# launch sequence faster than the GPU drains it, so a replay saves host time but no device time:
# on one MI355X a 68-frame streaming chunk took 2.31 ms either way, and config 3's packed
# groups 19.4 ms either way.  Small calls (streaming chunks) therefore launch eagerly.
HIFT_GRAPH_MIN_FRAMES = 1024


def capacity_bucket(frames: int, n_docs: int) -> tuple[int, int]:
    """The capacity a packed vocoder call of ``frames`` Mel frames in ``n_docs`` requests is
    run in: frames rounded up to m * 2^e with m in 8..15 (at most 12.5 % above, at least 64),
    requests to a power of two.  Calls in one bucket share its captured graph."""
    cap = 64
    while cap < frames:
        cap *= 2
    low = cap // 2
    for m in range(9, 17):
        if m * low // 8 >= frames:
            cap = max(64, m * low // 8)
            break
    docs = 1
    while docs < n_docs:
        docs *= 2
    return cap, docs


_BUFFER_SETS = 4  # per lane: one buffer set per vocoder graph its handle can pool


class HiFTVocoder:
    """Packed-batch HiFT vocoder on gfx950 HIP kernels (CausalHiFTGenerator counterpart)."""

    def __init__(self, dims: HiFTDims = HiFTDims(), device: torch.device | str = "cuda:0",
                 buffers: dict[str, torch.Tensor] | None = None):
        self.dims = dims
        self.device = torch.device(device)
        self.state: dict[str, torch.Tensor] | None = None
        self.buffers = buffers
        self._lib = _lib.load()
        self._cdims = self._make_dims()
        self._handle: int | None = None
        self._keep: list[torch.Tensor] = []
        # extra handles over the same weight table, for request groups in flight together:
        # [handle, workspace, stream]
        self._lanes: list[list] = []

    # ---- construction ----------------------------------------------------------------------

    def _make_dims(self) -> _lib.FcvHiftDims:
        d = self.dims
        c = _lib.FcvHiftDims()
        c.in_channels, c.base_channels, c.nb_harmonics = d.in_channels, d.base_channels, d.nb_harmonics
        c.sampling_rate = d.sampling_rate
        c.nsf_alpha, c.nsf_sigma, c.nsf_voiced_threshold = d.nsf_alpha, d.nsf_sigma, d.nsf_voiced_threshold
        c.n_stages = len(d.upsample_rates)
        for i, (r, k) in enumerate(zip(d.upsample_rates, d.upsample_kernel_sizes)):
            c.upsample_rates[i], c.upsample_kernels[i] = r, k
        c.n_kernels = len(d.resblock_kernel_sizes)
        c.n_dilations = len(d.resblock_dilation_sizes[0])
        for j, (k, dil) in enumerate(zip(d.resblock_kernel_sizes, d.resblock_dilation_sizes)):
            c.resblock_kernels[j] = k
            for m, v in enumerate(dil):
                c.resblock_dilations[j][m] = v
        for i, (k, dil) in enumerate(zip(d.source_resblock_kernel_sizes,
                                         d.source_resblock_dilation_sizes)):
            if len(dil) != c.n_dilations:
                raise ValueError("source and main resblocks must have the same dilation count")
            c.source_kernels[i] = k
            for m, v in enumerate(dil):
                c.source_dilations[i][m] = v
        c.n_fft, c.hop_len = d.n_fft, d.hop_len
        c.conv_pre_look_right, c.f0_channels = d.conv_pre_look_right, d.f0_channels
        c.lrelu_slope, c.audio_limit = d.lrelu_slope, d.audio_limit
        c.noise_samples = 0
        return c

    def load_reference_state_dict(self, sd: dict[str, torch.Tensor]) -> None:
        """Strict load of a ``hift.pt`` state dict (``generator.`` prefix optional)."""
        sd = {k[len("generator."):] if k.startswith("generator.") else k: v for k, v in sd.items()}
        want = dict(hift_state_dict_shapes(self.dims))
        missing = [k for k in want if k not in sd]
        unexpected = [k for k in sd if k not in want]
        if missing or unexpected:
            raise RuntimeError(f"HiFT state-dict mismatch: missing={missing[:8]}, "
                               f"unexpected={unexpected[:8]}")
        bad = [k for k, s in want.items() if tuple(sd[k].shape) != tuple(s)]
        if bad:
            raise RuntimeError(f"HiFT state-dict shape mismatch: {bad[:8]}")
        self.state = {k: v.detach().float().cpu() for k, v in sd.items()}

    def set_source_buffers(self, rand_ini: torch.Tensor, sine_waves: torch.Tensor) -> None:
        """The causal source's fixed buffers, e.g. a reference model's
        ``m_source.l_sin_gen.rand_ini`` [1, H] and ``.sine_waves`` [1, N, H]."""
        self.buffers = {"rand_ini": rand_ini, "sine_waves": sine_waves}

    @torch.no_grad()
    def finalize_weights(self) -> None:
        """Fold, pack and upload; create the library handle."""
        if self.state is None:
            raise RuntimeError("load_reference_state_dict() first")
        if self._handle is not None:
            raise RuntimeError("HiFTVocoder weights have already been finalized")
        if self.device.type != "cuda":
            raise ValueError("HiFTVocoder runs on a GPU device")
        d, sd, dev = self.dims, self.state, self.device
        H = d.nb_harmonics + 1
        keep: list[torch.Tensor] = []

        def put(t: torch.Tensor) -> int:
            t = t.contiguous().to(dev)
            keep.append(t)
            return t.data_ptr()

        def folded(name: str, dtype=torch.float32) -> torch.Tensor:
            if name + ".weight" in sd:
                return sd[name + ".weight"].to(dtype)
            g, v = sd[name + _G].to(dtype), sd[name + _V].to(dtype)
            norm = v.flatten(1).norm(dim=1).view(-1, 1, 1)
            return v * (g / norm)

        def conv(name: str, dtype=torch.float32, cin_pad: int | None = None) -> list[int]:
            w = folded(name, dtype)
            cout, cin, k = w.shape
            packed = torch.zeros(_ceil(cout, 64), k, cin_pad or _ceil(cin, 16), dtype=dtype)
            packed[:cout, :, :cin] = w.permute(0, 2, 1)
            return [put(packed), put(sd[name + ".bias"].to(dtype))]

        def snake(name: str) -> list[int]:
            a = sd[name + ".alpha"].float()
            return [put(a), put(1.0 / (a + 1e-9))]

        def resblock(name: str, n_dil: int) -> list[int]:
            out = []
            for j in range(n_dil):
                out += conv(f"{name}.convs1.{j}") + conv(f"{name}.convs2.{j}")
                out += snake(f"{name}.activations1.{j}") + snake(f"{name}.activations2.{j}")
            return out

        S = len(d.upsample_rates)
        K = len(d.resblock_kernel_sizes)
        D = len(d.resblock_dilation_sizes[0])
        ptrs = [put(sd["m_source.l_linear.weight"].reshape(H)), put(sd["m_source.l_linear.bias"])]
        ptrs += conv("conv_pre")
        for i in range(S):
            ptrs += conv(f"ups.{i}")
        for i in range(S):
            ptrs += conv(f"source_downs.{i}", cin_pad=32)
        for i in range(S):
            ptrs += resblock(f"source_resblocks.{i}", D)
        for i in range(S * K):
            ptrs += resblock(f"resblocks.{i}", D)
        ptrs += conv("conv_post")
        for i in (0, 2, 4, 6, 8):
            ptrs += conv(f"f0_predictor.condnet.{i}", torch.float64)
        ptrs += [put(sd["f0_predictor.classifier.weight"].double().reshape(-1)),
                 put(sd["f0_predictor.classifier.bias"].double())]
        window = torch.from_numpy(get_window("hann", d.n_fft, fftbins=True).astype(np.float32))
        buf = self.buffers or random_hift_buffers(d)
        table = buf["sine_waves"].reshape(-1, H).float()
        ptrs += [put(window), put(buf["rand_ini"].reshape(H).float()), put(table)]
        self._cdims.noise_samples = table.shape[0]
        n = int(self._lib.fcv_hift_weight_count(self._cdims))
        if n != len(ptrs):
            raise RuntimeError(f"weight table has {len(ptrs)} entries, the library expects {n}")
        arr = (_lib.c_void_p * n)(*ptrs)
        handle = _lib.c_void_p()
        _lib.check(self._lib.fcv_hift_create(self._cdims, arr, n, handle))
        self._handle = handle.value
        self._keep = keep
        self._ptrs = arr

    def __del__(self):
        try:
            for lane in getattr(self, "_lanes", [])[1:]:  # lane 0 is this vocoder's own handle
                self._lib.fcv_hift_destroy(lane[0])
            if getattr(self, "_handle", None) is not None:
                self._lib.fcv_hift_destroy(self._handle)
        except Exception:  # interpreter shutdown: the library may already be unloaded
            pass

    def _lane(self, i: int) -> list:
        """Request group i's [handle, workspace, stream]: group 0 is this vocoder's own handle;
        later groups get handles over the same weight table.  Group i runs on the process's
        group-i stream (streams.group_stream)."""
        self._require()
        while len(self._lanes) < i + 1:
            if not self._lanes:
                handle = self._handle
            else:
                h = _lib.c_void_p()
                _lib.check(self._lib.fcv_hift_create(self._cdims, self._ptrs, len(self._ptrs), h))
                handle = h.value
            # [handle, workspace, stream, buffer sets by capacity]
            self._lanes.append([handle, None, group_stream(self.device, len(self._lanes)), {}])
        return self._lanes[i]

    def _require(self) -> int:
        if self._handle is None:
            raise RuntimeError("call finalize_weights() before inference")
        return self._handle

    # ---- inference -------------------------------------------------------------------------

    def output_samples(self, frames: int, finalize: bool = True) -> int:
        n = int(self._lib.fcv_hift_output_samples(self._require(), int(frames), int(finalize)))
        if n < 0:
            raise ValueError(f"{frames} Mel frames are too few for a "
                             f"{'final' if finalize else 'non-final'} chunk")
        return n

    def graph_stats(self, group: int = 0) -> tuple[int, int]:
        """(vocoder graphs held, calls captured so far) of request group ``group``'s handle."""
        pooled, captures = _lib.c_int32(), _lib.c_int32()
        _lib.check(self._lib.fcv_hift_graph_stats(self._lane(group)[0], pooled, captures))
        return pooled.value, captures.value

    def _buffers(self, lane: list, cap: tuple[int, int], return_source: bool) -> dict:
        """The lane's input and output buffers for capacity ``cap`` (kept per capacity, so the
        pointers a captured graph was recorded with come back with its capacity)."""
        sets = lane[3]
        key = (cap, return_source)
        bufs = sets.pop(key, None)
        if bufs is None:
            frames, docs = cap
            scale = self.dims.upsample_scale
            f32 = lambda n: torch.empty(max(n, 1), dtype=torch.float32, device=self.device)
            bufs = {"mel": torch.zeros(frames, self.dims.in_channels, dtype=torch.float32,
                                       device=self.device),
                    "speech": f32(scale * frames + self.dims.hop_len * docs),
                    "source": f32(scale * frames) if return_source else None}
            while len(sets) >= _BUFFER_SETS:
                sets.pop(next(iter(sets)))
        sets[key] = bufs
        return bufs

    def _run(self, lane: list, mels: list[torch.Tensor], fin: list[bool], return_source: bool,
             stream: int, graph: bool | None = None) -> tuple[list, list]:
        """Packed calls of at most HIFT_MAX_DOCS requests on ``lane``, enqueued on ``stream``.
        Each call runs in its capacity bucket (``capacity_bucket``) from the lane's buffers for
        that capacity; with ``graph`` the capacity's captured graph replays it (None: for
        capacities of at least ``HIFT_GRAPH_MIN_FRAMES`` frames)."""
        h = lane[0]
        speech_all, source_all = [], []
        for g0 in range(0, len(mels), _lib.HIFT_MAX_DOCS):
            group = mels[g0:g0 + _lib.HIFT_MAX_DOCS]
            gfin = fin[g0:g0 + _lib.HIFT_MAX_DOCS]
            frames = [int(m.shape[1]) for m in group]
            samples = [self.output_samples(t, f) for t, f in zip(frames, gfin)]
            f0_frames = [t if f else t - 3 for t, f in zip(frames, gfin)]
            src_len = [t * self.dims.upsample_scale for t in f0_frames]
            cap = capacity_bucket(sum(frames), len(group))
            replay = graph if graph is not None else cap[0] >= HIFT_GRAPH_MIN_FRAMES
            bufs = self._buffers(lane, cap, return_source)
            off = 0
            for m in group:
                n = int(m.shape[1])
                bufs["mel"][off:off + n].copy_(m.to(self.device, torch.float32).transpose(0, 1))
                off += n
            fr = (_lib.c_int32 * len(group))(*frames)
            fl = (_lib.c_int32 * len(group))(*[int(f) for f in gfin])
            need = int(self._lib.fcv_hift_workspace_bytes_capacity(h, cap[0], cap[1]))
            if need == 0:
                raise ValueError("bad HiFT call layout")
            if lane[1] is None or lane[1].numel() < need:
                lane[1] = None
                lane[1] = torch.empty(need, dtype=torch.uint8, device=self.device)
            source = bufs["source"]
            _lib.check(self._lib.fcv_hift_inference_capacity(
                h, bufs["mel"].data_ptr(), fr, fl, len(group), cap[0], cap[1],
                bufs["speech"].data_ptr(), source.data_ptr() if source is not None else None,
                lane[1].data_ptr(), lane[1].numel(), int(bool(replay)), stream))
            # the buffers are the lane's: the next call writes them again
            speech = bufs["speech"][:sum(samples)].clone()
            off = 0
            for n in samples:
                speech_all.append(speech[off:off + n].view(1, n))
                off += n
            if source is not None:
                source = source[:sum(src_len)].clone()
                off = 0
                for n in src_len:
                    source_all.append(source[off:off + n].view(1, 1, n))
                    off += n
        return speech_all, source_all

    @torch.no_grad()
    def inference_batched(self, mels: Sequence[torch.Tensor],
                          finalize_list: Sequence[bool] | None = None,
                          return_source: bool = False, concurrency: int | None = None,
                          graph: bool | None = None):
        """Vocode requests of different lengths in packed passes.  ``mels``: each ``[80, T]``
        or ``[1, 80, T]``.  Returns one ``[1, N]`` fp32 waveform per request (and the
        ``[1, 1, L]`` sources with ``return_source``).  Each waveform equals what
        ``inference`` gives for that request alone.

        The requests run as ``concurrency`` groups (default: 2 when there are at least 2),
        balanced by Mel frames, each a packed call on its own handle over the shared weights
        and its own stream, all in flight together (one packed call of 8 requests at config 3:
        23.5 ms; two groups: 22.1 ms).

        Each call runs in a capacity bucket (``capacity_bucket``); with ``graph`` the launch
        sequence is captured on a bucket's second call and replayed for every later layout in
        it (fcv_hift_inference_capacity), bit-identical to an eager call.  ``graph=None`` (the
        default) replays for capacities of at least ``HIFT_GRAPH_MIN_FRAMES`` frames and
        launches smaller calls eagerly."""
        self._require()
        mels = [m.reshape(m.shape[-2], m.shape[-1]) for m in mels]
        if not mels:
            raise ValueError("no Mel input")
        fin = [True] * len(mels) if finalize_list is None else [bool(f) for f in finalize_list]
        if len(fin) != len(mels):
            raise ValueError("one finalize flag per request is required")
        n_groups = (2 if len(mels) >= 2 else 1) if concurrency is None else int(concurrency)
        if n_groups < 1:
            raise ValueError("concurrency must be >= 1")
        # longest first onto the group with the fewest frames
        groups: list[list[int]] = [[] for _ in range(min(n_groups, len(mels)))]
        load = [0] * len(groups)
        for i in sorted(range(len(mels)), key=lambda i: -int(mels[i].shape[1])):
            g = load.index(min(load))
            groups[g].append(i)
            load[g] += int(mels[i].shape[1])
        groups = [sorted(g) for g in groups]
        current = torch.cuda.current_stream(self.device)
        lanes = [self._lane(k) for k in range(len(groups))]
        for lane in lanes:  # every group waits for the caller's work only
            lane[2].wait_stream(current)
        results = []
        for lane, g in zip(lanes, groups):
            with torch.cuda.stream(lane[2]):
                results.append(self._run(lane, [mels[i] for i in g], [fin[i] for i in g],
                                         return_source, lane[2].cuda_stream, graph))
        for lane in lanes:
            current.wait_stream(lane[2])
        speech_all: list = [None] * len(mels)
        source_all: list = [None] * len(mels)
        for g, (sp, so) in zip(groups, results):
            for k, i in enumerate(g):
                sp[k].record_stream(current)
                speech_all[i] = sp[k]
                if return_source:
                    so[k].record_stream(current)
                    source_all[i] = so[k]
        return (speech_all, source_all) if return_source else speech_all

    @torch.no_grad()
    def inference(self, speech_feat: torch.Tensor, finalize: bool = True):
        """``CausalHiFTGenerator.inference(speech_feat, finalize)`` (generator.py:719-735):
        ``speech_feat`` ``[B, 80, T]`` -> (waveform ``[B, N]``, source ``[B, 1, L]``)."""
        if speech_feat.dim() != 3:
            raise ValueError("speech_feat must be [B, 80, T]")
        speech, source = self.inference_batched(list(speech_feat), [finalize] * speech_feat.shape[0],
                                                return_source=True)
        return torch.cat(speech), torch.cat(source)
