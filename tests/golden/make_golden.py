"""Write the golden vectors that pin the oracle's DiT wiring to the reference.

Run in the build container only (the reference tree is not present on GPU hosts):

    python tests/golden/make_golden.py [--ref /root/reference]

It imports the reference's own ``cosyvoice/flow/DiT/dit.py``, ``modules.py``,
``cosyvoice/utils/mask.py`` and ``flashinfer_flow.py`` (the module wiring of ``DiT.forward``,
``dit.py:145-176``, and ``solve_euler_batched``, ``flashinfer_flow.py:16-74``, are not fixed by
any closed form), feeds them seeded weights and inputs, and stores inputs + outputs as
``.npz`` fixtures next to this script.  Two packages the reference imports are not installed
here and are replaced by stubs registered in ``sys.modules`` before the import:

* ``torchaudio`` -- used only by ``MelSpec`` (modules.py:24-65), never by the DiT; the stub is
  an empty module;
* ``x_transformers`` 2.23.5 -- ``RotaryEmbedding`` / ``apply_rotary_pos_emb``; the stub restates
  the interleaved-pair rotation (the same arithmetic as the reference's Triton restatement,
  flashinfer_kernels.py:219-249).  The fixtures therefore pin everything except the
  x_transformers rotary arithmetic itself.

``hift_small.npz`` pins the wiring of the reference's ``CausalHiFTGenerator.inference``
(hifigan/generator.py:578-735 with f0_predictor.py:62-103): the order of the upsampling
stages, the source fusion, the resblock mean, the reflection pad and the two LeakyReLU slopes
are not fixed by any closed form.  The generator is built at a reduced width (base 32, two
stages) from its own source; our seeded weights are loaded into it with ``strict=True`` (which
also pins the ``hift.pt`` parameter names), and its fixed random buffers are stored with the
outputs.  ``--only hift`` writes just that file.

``prelookahead.npz`` pins the front-end oracle's ``pre_lookahead`` to the reference's own
``PreLookaheadLayer`` (cosyvoice/transformer/upsample_encoder.py:55-92) at the flow's shape
(builders.py:32-34: 80 -> 1024 -> 80, lookahead 3), with our seeded flow weights loaded
``strict=True``: a finalized padded batch of two sequences (zero right pad, one shorter than
the other) and the streaming form with a 3-frame right context (``flashinfer_flow.py:198-204``).
``--only frontend`` writes just that file.
"""

from __future__ import annotations

import argparse
import json
import sys
import types
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent


def _install_stubs() -> None:
    sys.modules.setdefault("torchaudio", types.ModuleType("torchaudio"))
    xt = types.ModuleType("x_transformers")
    xtx = types.ModuleType("x_transformers.x_transformers")

    class RotaryEmbedding(torch.nn.Module):
        def __init__(self, dim, base=10000.0):
            super().__init__()
            inv_freq = 1.0 / (base ** (torch.arange(0, dim, 2).float() / dim))
            self.register_buffer("inv_freq", inv_freq)

        def forward_from_seq_len(self, seq_len):
            t = torch.arange(seq_len, device=self.inv_freq.device)
            return self.forward(t)

        def forward(self, t):
            if t.ndim == 1:
                t = t[None]
            freqs = torch.einsum("bi,j->bij", t.type_as(self.inv_freq), self.inv_freq)
            freqs = torch.stack((freqs, freqs), dim=-1).flatten(-2)
            return freqs, 1.0

    def _rotate_half(x):
        x = x.reshape(*x.shape[:-1], x.shape[-1] // 2, 2)
        x1, x2 = x.unbind(-1)
        return torch.stack((-x2, x1), dim=-1).flatten(-2)

    def apply_rotary_pos_emb(t, freqs, scale=1):
        rot_dim, seq_len = freqs.shape[-1], t.shape[-2]
        freqs = freqs[:, -seq_len:, :]
        if t.ndim == 4 and freqs.ndim == 3:
            freqs = freqs[:, None]
        head, rest = t[..., :rot_dim], t[..., rot_dim:]
        head = head * freqs.cos() * scale + _rotate_half(head) * freqs.sin() * scale
        return torch.cat((head, rest), dim=-1).type(t.dtype)

    xtx.RotaryEmbedding = RotaryEmbedding
    xtx.apply_rotary_pos_emb = apply_rotary_pos_emb
    xt.x_transformers = xtx
    sys.modules.setdefault("x_transformers", xt)
    sys.modules.setdefault("x_transformers.x_transformers", xtx)


def _synthetic():
    import importlib.util
    name = "faster_cosyvoice_amd"
    pkg_dir = REPO / "faster-cosyvoice_amd"
    spec = importlib.util.spec_from_file_location(f"{name}_synthetic", pkg_dir / "synthetic.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod
    spec.loader.exec_module(mod)
    return mod


def _inputs(rng, B, T, lengths):
    x = rng.standard_normal((B, 80, T)).astype(np.float32)
    mu = rng.standard_normal((B, 80, T)).astype(np.float32)
    cond = rng.standard_normal((B, 80, T)).astype(np.float32)
    spks = rng.standard_normal((B, 80)).astype(np.float32)
    t = rng.uniform(0, 1, size=(B,)).astype(np.float32)
    mask = np.zeros((B, 1, T), np.float32)
    for b, n in enumerate(lengths):
        mask[b, 0, :n] = 1
        cond[b, :, n:] = 0
    return dict(x=x, mu=mu, cond=cond, spks=spks, t=t, mask=mask)


HIFT_SMALL = dict(base_channels=32, upsample_rates=(2, 3), upsample_kernel_sizes=(4, 5),
                  resblock_kernel_sizes=(3, 5), resblock_dilation_sizes=((1, 2), (1, 3)),
                  source_resblock_kernel_sizes=(3, 5), source_resblock_dilation_sizes=((1, 2), (1, 2)),
                  f0_channels=16)


def hift_golden() -> None:
    """A reduced-width CausalHiFTGenerator on seeded Mel, finalize True and False."""
    from faster_cosyvoice.token2wav.cosyvoice.hifigan.f0_predictor import (  # noqa: E402
        CausalConvRNNF0Predictor)
    from faster_cosyvoice.token2wav.cosyvoice.hifigan.generator import (  # noqa: E402
        CausalHiFTGenerator)

    syn = _synthetic()
    torch.set_grad_enabled(False)
    dims = syn.HiFTDims(**HIFT_SMALL)
    sd = syn.random_hift_state_dict(dims, seed=61)
    torch.manual_seed(62)  # the generator draws its fixed source buffers at construction
    model = CausalHiFTGenerator(
        in_channels=80, base_channels=dims.base_channels, nb_harmonics=dims.nb_harmonics,
        sampling_rate=dims.sampling_rate, nsf_alpha=dims.nsf_alpha, nsf_sigma=dims.nsf_sigma,
        nsf_voiced_threshold=dims.nsf_voiced_threshold,
        upsample_rates=list(dims.upsample_rates),
        upsample_kernel_sizes=list(dims.upsample_kernel_sizes),
        istft_params={"n_fft": dims.n_fft, "hop_len": dims.hop_len},
        resblock_kernel_sizes=list(dims.resblock_kernel_sizes),
        resblock_dilation_sizes=[list(d) for d in dims.resblock_dilation_sizes],
        source_resblock_kernel_sizes=list(dims.source_resblock_kernel_sizes),
        source_resblock_dilation_sizes=[list(d) for d in dims.source_resblock_dilation_sizes],
        lrelu_slope=dims.lrelu_slope, audio_limit=dims.audio_limit,
        conv_pre_look_right=dims.conv_pre_look_right,
        f0_predictor=CausalConvRNNF0Predictor(num_class=1, in_channels=80,
                                              cond_channels=dims.f0_channels))
    model.load_state_dict(sd, strict=True)
    model.eval()
    rng = np.random.Generator(np.random.PCG64(63))
    T = 24
    mel = torch.from_numpy(rng.standard_normal((1, 80, T)).astype(np.float32))
    out = {}
    for fin in (True, False):
        f0 = model.f0_predictor.to(torch.float64)(mel.double(), finalize=fin)
        speech, s = model.inference(speech_feat=mel, finalize=fin)
        tag = "fin" if fin else "stream"
        out.update({f"f0_{tag}": f0.numpy(), f"speech_{tag}": speech.numpy(), f"s_{tag}": s.numpy()})
    L = T * dims.upsample_scale
    gen = model.m_source.l_sin_gen
    np.savez_compressed(
        HERE / "hift_small.npz", mel=mel.numpy(), weight_seed=np.int32(61),
        config=np.array(json.dumps(HIFT_SMALL)),
        rand_ini=gen.rand_ini.numpy(), sine_waves=gen.sine_waves[:, :L].numpy(), **out)


def frontend_golden() -> None:
    """The reference's PreLookaheadLayer at the flow's shape, finalized and with context."""
    from faster_cosyvoice.token2wav.cosyvoice.transformer.upsample_encoder import (  # noqa: E402
        PreLookaheadLayer)

    syn = _synthetic()
    torch.set_grad_enabled(False)
    dims = syn.FlowDims()
    sd = syn.random_flow_state_dict(dims, seed=71)
    layer = PreLookaheadLayer(in_channels=dims.feat, channels=dims.channels,
                              pre_lookahead_len=dims.lookahead)
    prefix = "pre_lookahead_layer."
    layer.load_state_dict({k[len(prefix):]: v for k, v in sd.items() if k.startswith(prefix)},
                          strict=True)
    layer.eval()
    rng = np.random.Generator(np.random.PCG64(72))
    x = rng.standard_normal((2, 13, dims.feat)).astype(np.float32)
    x[1, 9:] = 0.0  # the second sequence is 9 frames long, zero-padded as the flow's mask leaves it
    out_final = layer(torch.from_numpy(x))
    xs = rng.standard_normal((1, 10, dims.feat)).astype(np.float32)
    ctx = rng.standard_normal((1, dims.lookahead, dims.feat)).astype(np.float32)
    out_ctx = layer(torch.from_numpy(xs), torch.from_numpy(ctx))
    np.savez_compressed(HERE / "prelookahead.npz", weight_seed=np.int32(71),
                        lookahead=np.int32(dims.lookahead), x=x, out_final=out_final.numpy(),
                        x_stream=xs, context=ctx, out_context=out_ctx.numpy())


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    ap.add_argument("--only", choices=["hift", "frontend"], default=None)
    args = ap.parse_args()
    _install_stubs()
    sys.path.insert(0, args.ref)
    if args.only == "hift":
        hift_golden()
        print("wrote hift_small.npz")
        return
    if args.only == "frontend":
        frontend_golden()
        print("wrote prelookahead.npz")
        return
    from faster_cosyvoice.token2wav.cosyvoice.flow.DiT.dit import DiT  # noqa: E402
    from faster_cosyvoice.token2wav.flashinfer_flow import solve_euler_batched  # noqa: E402

    syn = _synthetic()
    torch.set_grad_enabled(False)

    # ---- tiny DiT: dim 128, depth 2, 2 heads x 64, padded batch of 2 ---------------------
    dims = syn.DiTDims(dim=128, depth=2, heads=2, dim_head=64, ff_mult=2)
    sd = syn.random_state_dict(dims, seed=11, gate_bias=0.5)
    model = DiT(dim=128, depth=2, heads=2, dim_head=64, ff_mult=2, mel_dim=80, mu_dim=80,
                spk_dim=80, out_channels=80, static_chunk_size=8, num_decoding_left_chunks=-1)
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected and all("rotary" in k for k in missing), (missing, unexpected)
    model.eval()
    rng = np.random.Generator(np.random.PCG64(2024))
    lengths = [40, 29]
    inp = _inputs(rng, 2, 40, lengths)
    tt = {k: torch.from_numpy(v) for k, v in inp.items()}
    out_full = model(tt["x"], tt["mask"], tt["mu"], tt["t"], tt["spks"], tt["cond"], streaming=False)
    out_stream = model(tt["x"], tt["mask"], tt["mu"], tt["t"], tt["spks"], tt["cond"], streaming=True)

    decoder = types.SimpleNamespace(
        inference_cfg_rate=0.7,
        forward_estimator=lambda x, mask, mu, t, spks, cond, streaming: model(
            x, mask, mu, t, spks, cond, streaming=streaming))
    sample = solve_euler_batched(decoder, tt["x"], tt["mu"], tt["mask"], tt["spks"], tt["cond"],
                                 num_timesteps=4, streaming=False)
    np.savez_compressed(
        HERE / "tiny_dit.npz", **inp, lengths=np.array(lengths, np.int32), chunk=np.int32(8),
        weight_seed=np.int32(11), gate_bias=np.float32(0.5), dim=np.int32(128), depth=np.int32(2),
        heads=np.int32(2), out_full=out_full.numpy(), out_stream=out_stream.numpy(),
        euler_steps=np.int32(4), euler_cfg=np.float32(0.7), euler_sample=sample.float().numpy())

    # ---- one full-size block: dim 1024, 16 heads, 64 frames, streaming chunk 50 ---------
    dims = syn.DiTDims(dim=1024, depth=1)
    sd = syn.random_state_dict(dims, seed=5, gate_bias=0.5)
    model = DiT(dim=1024, depth=1, heads=16, dim_head=64, ff_mult=2, mel_dim=80, mu_dim=80,
                spk_dim=80, out_channels=80, static_chunk_size=50, num_decoding_left_chunks=-1)
    model.load_state_dict(sd, strict=False)
    model.eval()
    rng = np.random.Generator(np.random.PCG64(77))
    inp = _inputs(rng, 1, 64, [64])
    tt = {k: torch.from_numpy(v) for k, v in inp.items()}
    out_full = model(tt["x"], tt["mask"], tt["mu"], tt["t"], tt["spks"], tt["cond"], streaming=False)
    out_stream = model(tt["x"], tt["mask"], tt["mu"], tt["t"], tt["spks"], tt["cond"], streaming=True)
    np.savez_compressed(
        HERE / "block1024.npz", **inp, lengths=np.array([64], np.int32), chunk=np.int32(50),
        weight_seed=np.int32(5), gate_bias=np.float32(0.5), dim=np.int32(1024), depth=np.int32(1),
        heads=np.int32(16), out_full=out_full.numpy(), out_stream=out_stream.numpy())
    hift_golden()
    frontend_golden()
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
