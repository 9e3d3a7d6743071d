"""``DiTEstimator``: the MI355X drop-in for the reference's ``FlashInferDiT``.

Same state-dict layout as the CosyVoice3 DiT (``cosyvoice/flow/DiT/dit.py:104-143``, as
``FlashInferDiT`` keeps it, ``flashinfer_dit.py:5-7,163-179``), same call
``forward(x, mask, mu, t, spks, cond, streaming=False)`` (``flashinfer_dit.py:315-362``),
same packed CFG layout.  All compute runs in libfcvdit.so; the torch modules below only hold
parameters so that ``load_state_dict`` of a ``flow.pt`` decoder estimator works unchanged.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch
import torch.nn as nn

from . import _lib
from .synthetic import DiTDims

ROPE_MAX_POS = 8192
TEMB_FREQ = 256


# ---- parameter holders with the reference's module names -----------------------------------


class _TimestepEmbedding(nn.Module):
    def __init__(self, dim: int, device):
        super().__init__()
        self.time_mlp = nn.Sequential(nn.Linear(TEMB_FREQ, dim, device=device), nn.SiLU(),
                                      nn.Linear(dim, dim, device=device))


class _CausalConvPositionEmbedding(nn.Module):
    def __init__(self, dim: int, kernel_size: int, groups: int, device):
        super().__init__()
        self.kernel_size = kernel_size
        self.conv1 = nn.Sequential(nn.Conv1d(dim, dim, kernel_size, groups=groups, device=device),
                                   nn.Mish())
        self.conv2 = nn.Sequential(nn.Conv1d(dim, dim, kernel_size, groups=groups, device=device),
                                   nn.Mish())


class _InputEmbedding(nn.Module):
    def __init__(self, in_dim: int, dim: int, kernel_size: int, groups: int, device):
        super().__init__()
        self.proj = nn.Linear(in_dim, dim, device=device)
        self.conv_pos_embed = _CausalConvPositionEmbedding(dim, kernel_size, groups, device)


class _AdaNorm(nn.Module):
    def __init__(self, dim: int, chunks: int, device):
        super().__init__()
        self.linear = nn.Linear(dim, chunks * dim, device=device)


class _Attention(nn.Module):
    def __init__(self, dim: int, inner: int, device):
        super().__init__()
        self.to_q = nn.Linear(dim, inner, device=device)
        self.to_k = nn.Linear(dim, inner, device=device)
        self.to_v = nn.Linear(dim, inner, device=device)
        self.to_out = nn.ModuleList([nn.Linear(inner, dim, device=device), nn.Dropout(0.0)])


class _FeedForward(nn.Module):
    def __init__(self, dim: int, inner: int, device):
        super().__init__()
        self.ff = nn.Sequential(
            nn.Sequential(nn.Linear(dim, inner, device=device), nn.GELU(approximate="tanh")),
            nn.Dropout(0.0), nn.Linear(inner, dim, device=device))


class _Block(nn.Module):
    def __init__(self, dim: int, heads: int, dim_head: int, ff_dim: int, device):
        super().__init__()
        self.attn_norm = _AdaNorm(dim, 6, device)
        self.attn = _Attention(dim, heads * dim_head, device)
        self.ff = _FeedForward(dim, ff_dim, device)


# ---- one library handle: workspace, packed-layout plan, launch stream ---------------------------


class _PackedRunner:
    """A libfcvdit handle with its own workspace, plan cache and launch stream.

    The estimator is one (request group 0); ``_Lane`` objects are more handles over the same
    derived weights, so that independent groups of requests can run on concurrent streams.
    Subclasses set ``device``, ``static_chunk_size`` and ``_handle``."""

    def _init_runner(self, group: int = 0) -> None:
        self._workspace: torch.Tensor | None = None
        self._plan_key: tuple | None = None
        self.group = group  # request group this runner serves (its stream: streams.group_stream)
        self.plan_calls = 0

    def _require(self) -> int:
        if self._handle is None:
            raise RuntimeError("call finalize_weights() before running the estimator")
        return self._handle

    def plan(self, seqlens: Sequence[int], streaming: bool = False,
             capacity: tuple[int, int] | None = None) -> None:
        """Plan the packed layout (FlashInfer ``plan`` equivalent); no-op when unchanged.

        ``capacity = (rows_cap, docs_cap)`` plans the layout inside that capacity
        (``fcv_dit_plan_capacity``): every layout planned into one capacity shares the solve
        graphs captured for it; None plans exactly this layout."""
        handle = self._require()
        lengths = tuple(int(n) for n in seqlens)
        key = (lengths, bool(streaming), capacity)
        if key == self._plan_key:
            return
        lib = _lib.load()
        rows = sum(lengths)
        rows_cap, docs_cap = capacity if capacity is not None else (rows, len(lengths))
        if rows > rows_cap or len(lengths) > docs_cap:
            raise ValueError(f"{rows} rows in {len(lengths)} documents exceed the capacity "
                             f"({rows_cap}, {docs_cap})")
        need = lib.fcv_dit_workspace_bytes(handle, rows_cap, docs_cap)
        if self._workspace is None or self._workspace.numel() < need:
            cap = max(need, 2 * (0 if self._workspace is None else self._workspace.numel()))
            self._workspace = None
            self._workspace = torch.empty(cap + 256, dtype=torch.uint8, device=self.device)
        base = self._workspace.data_ptr()
        aligned = (base + 255) // 256 * 256
        cu = [0]
        for n in lengths:
            cu.append(cu[-1] + n)
        cu_arr = (_lib.c_int32 * len(cu))(*cu)
        mode = _lib.FCV_MASK_CHUNK_CAUSAL if streaming else _lib.FCV_MASK_FULL
        _lib.check(lib.fcv_dit_plan_capacity(handle, cu_arr, len(lengths), mode,
                                             self.static_chunk_size, rows_cap, docs_cap, aligned,
                                             self._workspace.numel() - (aligned - base),
                                             self._stream_ptr()))
        self._plan_key = key
        self.plan_calls += 1

    def graph_stats(self) -> tuple[int, int]:
        """(solve graphs held, solves captured so far) of this runner's handle."""
        pooled, captures = _lib.c_int32(), _lib.c_int32()
        _lib.check(_lib.load().fcv_dit_graph_stats(self._require(), pooled, captures))
        return pooled.value, captures.value

    def _stream_ptr(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream


class _Lane(_PackedRunner):
    """A second handle over an estimator's derived weights (which the estimator keeps alive)."""

    def __init__(self, owner: "DiTEstimator", handle: int, group: int):
        self.device = owner.device
        self.static_chunk_size = owner.static_chunk_size
        self.dims = owner.dims
        self._handle = handle
        self._owner = owner
        self._init_runner(group)

    def __del__(self):
        handle = getattr(self, "_handle", None)
        lib = getattr(_lib, "_LIB", None) if _lib is not None else None
        if handle is not None and lib is not None:
            lib.fcv_dit_destroy(handle)
            self._handle = None


# ---- the estimator ----------------------------------------------------------------------------


class DiTEstimator(nn.Module, _PackedRunner):
    """Packed-batch CosyVoice3 DiT estimator on gfx950 HIP kernels.

    Mirrors ``FlashInferDiT`` (flashinfer_dit.py:98-186): construct, ``load_state_dict``,
    ``finalize_weights()`` once, then call it like the reference estimator.  Not re-entrant
    (one instance per GPU thread), like the reference.

    Args:
      dim, depth, heads, dim_head, ff_mult, mel_dim: DiT shape (builders.py:17-21).
      static_chunk_size: chunk of the streaming chunk-causal mask, in mel frames.
      device: the GPU that holds the derived weights and runs the kernels.
      rope_dim: flat q/k columns that RoPE rotates (64 = head 0, flashinfer_dit.py:61).
      max_pos: longest document the RoPE tables cover.
    """

    def __init__(self, dim: int = 1024, depth: int = 22, heads: int = 16, dim_head: int = 64,
                 ff_mult: int = 2, mel_dim: int = 80, mu_dim: int = 80, spk_dim: int = 80,
                 out_channels: int = 80, static_chunk_size: int = 50,
                 device: torch.device | str = "cuda:0", rope_dim: int = 64,
                 max_pos: int = ROPE_MAX_POS, param_device: torch.device | str = "meta") -> None:
        super().__init__()
        if mu_dim != mel_dim or spk_dim != mel_dim or out_channels != mel_dim:
            raise ValueError("mel_dim, mu_dim, spk_dim and out_channels must be equal")
        self.dims = DiTDims(dim=dim, depth=depth, heads=heads, dim_head=dim_head, ff_mult=ff_mult,
                            mel_dim=mel_dim)
        self.dim, self.depth, self.heads, self.dim_head = dim, depth, heads, dim_head
        self.out_channels = out_channels
        self.static_chunk_size = static_chunk_size
        self.rope_dim = rope_dim
        self.max_pos = max_pos
        self.device = torch.device(device)
        d = self.dims
        self.time_embed = _TimestepEmbedding(dim, param_device)
        self.input_embed = _InputEmbedding(d.in_dim, dim, d.conv_kernel, d.conv_groups,
                                           param_device)
        self.transformer_blocks = nn.ModuleList(
            [_Block(dim, heads, dim_head, d.ff_dim, param_device) for _ in range(depth)])
        self.norm_out = _AdaNorm(dim, 2, param_device)
        self.proj_out = nn.Linear(dim, mel_dim, device=param_device)

        self._handle: int | None = None
        self._derived: dict[str, torch.Tensor] = {}
        self._create_args: tuple | None = None
        self._extra_lanes: list[_Lane] = []
        self._init_runner()

    # -- loading ----------------------------------------------------------------------------

    @classmethod
    def from_state_dict(cls, state_dict: dict[str, torch.Tensor], device="cuda:0",
                        depth: int | None = None, **kwargs) -> "DiTEstimator":
        """Build with the state dict's depth, load it (assign, strict) and finalize."""
        if depth is None:
            depth = 0
            while f"transformer_blocks.{depth}.attn.to_q.weight" in state_dict:
                depth += 1
        model = cls(depth=depth, device=device, **kwargs)
        model.load_reference_state_dict(state_dict)
        model.finalize_weights()
        return model

    def load_reference_state_dict(self, state_dict: dict[str, torch.Tensor]) -> None:
        """``load_state_dict`` that tolerates only RoPE buffers as extra/missing keys
        (the reference's rule, flashinfer_dit.py:975-983)."""
        sd = {k: v for k, v in state_dict.items() if "rotary_embed" not in k and "rope" not in k}
        missing, unexpected = self.load_state_dict(sd, strict=False, assign=True)
        bad = [k for k in list(missing) + list(unexpected) if "rope" not in k]
        if bad:
            raise RuntimeError(f"state dict mismatch: {bad[:8]}")

    # -- weight derivation ------------------------------------------------------------------

    @torch.no_grad()
    def finalize_weights(self) -> None:
        """Derive the kernel-layout fp16 weights once (flashinfer_dit.py:228-313); fp16 is the
        dtype the reference's apply_flashinfer gives the DiT (flashinfer_dit.py:963).

        Fused QKV per block; "+1" folded into the AdaLN scale biases (chunks 1 and 4 of every
        block, chunk 0 of the final (scale, shift) pair); all AdaLN projections concatenated
        into one matrix; conv weights (C, C/G, K) re-laid out as (G, K, co, ci); proj_out padded
        to 128 rows; RoPE cos/sin tables in fp32 from the x_transformers angles.
        """
        if self._handle is not None:
            raise RuntimeError("DiTEstimator weights have already been finalized")
        if self.device.type != "cuda":
            raise ValueError("DiTEstimator runs on a GPU device")
        lib = _lib.load()
        dev, D, L = self.device, self.dim, self.depth
        h16 = lambda t: t.detach().to(device=dev, dtype=torch.float16).contiguous()
        f32 = lambda t: t.detach().to(device=dev, dtype=torch.float32).contiguous()
        blocks = self.transformer_blocks

        out: dict[str, torch.Tensor] = {}
        out["temb_w1"] = h16(self.time_embed.time_mlp[0].weight)
        out["temb_b1"] = f32(self.time_embed.time_mlp[0].bias)
        out["temb_w2"] = h16(self.time_embed.time_mlp[2].weight)
        out["temb_b2"] = f32(self.time_embed.time_mlp[2].bias)

        ada_w = [b.attn_norm.linear.weight for b in blocks] + [self.norm_out.linear.weight]
        out["ada_w"] = h16(torch.cat([w.detach().float().cpu() for w in ada_w]))
        ada_b = []
        for b in blocks:
            bias = b.attn_norm.linear.bias.detach().float().cpu().clone().view(6, D)
            bias[1] += 1.0
            bias[4] += 1.0
            ada_b.append(bias.reshape(-1))
        fin = self.norm_out.linear.bias.detach().float().cpu().clone().view(2, D)
        fin[0] += 1.0
        ada_b.append(fin.reshape(-1))
        out["ada_b"] = f32(torch.cat(ada_b))

        out["in_w"] = h16(self.input_embed.proj.weight)
        out["in_b"] = f32(self.input_embed.proj.bias)
        groups = self.dims.conv_groups
        cpg = D // groups
        for i, seq in enumerate((self.input_embed.conv_pos_embed.conv1,
                                 self.input_embed.conv_pos_embed.conv2), start=1):
            w = seq[0].weight.detach().float().cpu()  # (C, C/G, K)
            taps = w.shape[-1]
            w = w.view(groups, cpg, cpg, taps).permute(0, 3, 1, 2)  # (G, K, co, ci)
            out[f"conv{i}_w"] = h16(w.contiguous())
            out[f"conv{i}_b"] = f32(seq[0].bias)

        out["qkv_w"] = h16(torch.stack([torch.cat([b.attn.to_q.weight, b.attn.to_k.weight,
                                                  b.attn.to_v.weight]).detach().float().cpu()
                                       for b in blocks]))
        out["qkv_b"] = f32(torch.stack([torch.cat([b.attn.to_q.bias, b.attn.to_k.bias,
                                                   b.attn.to_v.bias]).detach().float().cpu()
                                        for b in blocks]))
        out["out_w"] = h16(torch.stack([b.attn.to_out[0].weight.detach().float().cpu() for b in blocks]))
        out["out_b"] = f32(torch.stack([b.attn.to_out[0].bias.detach().float().cpu() for b in blocks]))
        out["ff1_w"] = h16(torch.stack([b.ff.ff[0][0].weight.detach().float().cpu() for b in blocks]))
        out["ff1_b"] = f32(torch.stack([b.ff.ff[0][0].bias.detach().float().cpu() for b in blocks]))
        out["ff2_w"] = h16(torch.stack([b.ff.ff[2].weight.detach().float().cpu() for b in blocks]))
        out["ff2_b"] = f32(torch.stack([b.ff.ff[2].bias.detach().float().cpu() for b in blocks]))

        mel = self.dims.mel_dim
        pw = torch.zeros(128, D)
        pw[:mel] = self.proj_out.weight.detach().float().cpu()
        pb = torch.zeros(128)
        pb[:mel] = self.proj_out.bias.detach().float().cpu()
        out["proj_w"] = h16(pw)
        out["proj_b"] = f32(pb)

        cos, sin = rope_tables(self.max_pos, self.dim_head, self.rope_dim)
        out["rope_cos"] = f32(cos)
        out["rope_sin"] = f32(sin)

        dims = _lib.FcvDitDims(dim=D, depth=L, heads=self.heads, dim_head=self.dim_head,
                               ff_dim=self.dims.ff_dim, mel_dim=mel,
                               conv_kernel=self.dims.conv_kernel, conv_groups=groups,
                               rope_dim=self.rope_dim, max_pos=self.max_pos)
        weights = _lib.FcvDitWeights(**{k: out[k].data_ptr() for k in _lib.WEIGHT_FIELDS})
        handle = _lib.c_void_p()
        _lib.check(lib.fcv_dit_create(dims, weights, handle))
        self._handle = handle.value
        self._derived = out
        self._create_args = (dims, weights)
        # the derived copies are the only ones the kernels read; free the parameter storage
        for p in self.parameters():
            p.data = torch.empty(0)

    def __del__(self):
        handle = getattr(self, "_handle", None)
        lib = getattr(_lib, "_LIB", None) if _lib is not None else None
        if handle is not None and lib is not None:  # module globals may be gone at exit
            lib.fcv_dit_destroy(handle)
            self._handle = None

    # -- concurrent lanes -------------------------------------------------------------------

    def lanes(self, n: int) -> list[_PackedRunner]:
        """``n`` runners over this estimator's weights: the estimator itself, then extra
        handles created on first use (each with its own workspace, plan and stream)."""
        lib = _lib.load()
        self._require()
        while len(self._extra_lanes) < n - 1:
            handle = _lib.c_void_p()
            _lib.check(lib.fcv_dit_create(*self._create_args, handle))
            self._extra_lanes.append(_Lane(self, handle.value, len(self._extra_lanes) + 1))
        return [self] + self._extra_lanes[: n - 1]

    # -- compute ----------------------------------------------------------------------------

    @torch.no_grad()
    def forward_packed(self, x: torch.Tensor, mu: torch.Tensor, cond: torch.Tensor,
                       spks: torch.Tensor, t: torch.Tensor, seqlens: Sequence[int],
                       streaming: bool = False) -> torch.Tensor:
        """Velocity for packed rows.  x, mu, cond: [R, mel]; spks: [N, mel]; t: [N] or [1]."""
        handle = self._require()
        self.plan(seqlens, streaming)
        mel = self.dims.mel_dim
        rows = sum(int(n) for n in seqlens)
        conv = lambda a: a.to(device=self.device, dtype=torch.float32).contiguous()
        x, mu, cond, spks = conv(x), conv(mu), conv(cond), conv(spks)
        t = conv(t.reshape(-1))
        if x.shape != (rows, mel) or mu.shape != (rows, mel) or cond.shape != (rows, mel):
            raise ValueError(f"x, mu, cond must be [{rows}, {mel}]")
        if spks.shape != (len(seqlens), mel):
            raise ValueError(f"spks must be [{len(seqlens)}, {mel}]")
        out = torch.empty(rows, mel, dtype=torch.float32, device=self.device)
        _lib.check(_lib.load().fcv_dit_forward(handle, x.data_ptr(), mu.data_ptr(), cond.data_ptr(),
                                               spks.data_ptr(), t.data_ptr(), t.numel(),
                                               out.data_ptr(), self._stream_ptr()))
        return out

    @torch.no_grad()
    def forward(self, x: torch.Tensor, mask: torch.Tensor, mu: torch.Tensor, t: torch.Tensor,
                spks: torch.Tensor | None = None, cond: torch.Tensor | None = None,
                streaming: bool = False) -> torch.Tensor:
        """Reference estimator call (flashinfer_dit.py:315-362): padded ``[B,80,T]`` in and
        out, document lengths from ``mask[:,0].sum(-1)``, padded frames of the output zero."""
        if spks is None or cond is None:
            raise ValueError("spks and cond are required")
        handle = self._require()
        lib = _lib.load()
        batch, mel, padded = x.shape
        lengths = [int(v) for v in mask[:, 0].sum(-1).round().to(torch.int64).tolist()]
        self.plan(lengths, streaming)
        rows = sum(lengths)
        dev = self.device
        f32 = lambda a: a.to(device=dev, dtype=torch.float32).contiguous()
        stream = self._stream_ptr()
        packed = {}
        for name, src in (("x", x), ("mu", mu), ("cond", cond)):
            dst = torch.empty(rows, mel, dtype=torch.float32, device=dev)
            _lib.check(lib.fcv_pack_padded(handle, f32(src).data_ptr(), batch, mel, padded,
                                           dst.data_ptr(), stream))
            packed[name] = dst
        t = f32(t).reshape(-1)
        # the packed solver hands every document the same t (flashinfer_flow.py:53-57): one
        # modulation row then serves all of them (bit-identical to one row per document)
        if t.numel() > 1 and bool((t == t[0]).all()):
            t = t[:1]
        spk = f32(spks).reshape(batch, mel)
        v = torch.empty(rows, mel, dtype=torch.float32, device=dev)
        _lib.check(lib.fcv_dit_forward(handle, packed["x"].data_ptr(), packed["mu"].data_ptr(),
                                       packed["cond"].data_ptr(), spk.data_ptr(), t.data_ptr(),
                                       t.numel(), v.data_ptr(), stream))
        out = torch.empty(batch, mel, padded, dtype=torch.float32, device=dev)
        _lib.check(lib.fcv_unpack_padded(handle, v.data_ptr(), batch, mel, padded, out.data_ptr(),
                                         stream))
        return out.to(x.dtype)


def rope_tables(max_pos: int, dim_head: int = 64, rope_dim: int = 64,
                base: float = 10000.0) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin of the interleaved-pair angles ``p * base^(-2i/dim_head)``, fp32 arithmetic as
    the reference builds its tables (flashinfer_dit.py:262-273): ``[max_pos, rope_dim/2]``."""
    inv_freq = 1.0 / (base ** (torch.arange(0, dim_head, 2, dtype=torch.float32) / dim_head))
    pos = torch.arange(max_pos, dtype=torch.float32)
    theta = pos[:, None] * inv_freq[None, : rope_dim // 2]
    return theta.cos().contiguous(), theta.sin().contiguous()
