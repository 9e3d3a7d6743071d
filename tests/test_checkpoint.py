"""CPU checks of the ``flow.pt`` loader's host side (checkpoint.py): the key split, shape
inference, strict rejection of foreign keys, and the reference's fixed noise prefix."""

from __future__ import annotations

import pytest
import torch


def _flow_state_dict(fcv, depth=2):
    """A state dict with the key layout of the reference's CausalMaskedDiffWithDiT
    (flow.py:307-310 front-end names, the DiT under decoder.estimator., its RoPE buffer)."""
    syn = fcv.synthetic
    sd = syn.random_flow_state_dict(syn.FlowDims(vocab=33, channels=128), seed=1)
    dit = syn.random_state_dict(syn.DiTDims(dim=128, depth=depth, heads=2), seed=2)
    sd.update({"decoder.estimator." + k: v for k, v in dit.items()})
    sd["decoder.estimator.rotary_embed.inv_freq"] = torch.ones(32)
    return sd


def test_split_and_shapes_from_a_saved_file(fcv, tmp_path):
    from faster_cosyvoice_amd import checkpoint as ck
    path = tmp_path / "flow.pt"
    torch.save(_flow_state_dict(fcv, depth=3), path)
    sd = torch.load(path, map_location="cpu", weights_only=True)
    front, est = ck.split_flow_state_dict(sd)
    assert set(front) == {k for k, _ in fcv.synthetic.flow_state_dict_shapes()}
    assert "transformer_blocks.2.ff.ff.2.bias" in est and "rotary_embed.inv_freq" in est
    s = ck.flow_shapes(front, est)
    assert s == dict(vocab=33, feat=80, channels=128, lookahead=3, spk_dim=192, depth=3,
                     dim=128, heads=2, dim_head=64, ff_mult=2, mel=80)


def test_foreign_and_missing_keys_are_rejected(fcv):
    from faster_cosyvoice_amd import checkpoint as ck
    sd = _flow_state_dict(fcv)
    with pytest.raises(RuntimeError, match="unexpected"):
        ck.split_flow_state_dict({**sd, "encoder.layers.0.weight": torch.zeros(1)})
    front_only = {k: v for k, v in sd.items() if not k.startswith("decoder.")}
    with pytest.raises(RuntimeError, match="needs"):
        ck.split_flow_state_dict(front_only)
    gap = {k: v for k, v in sd.items() if ".transformer_blocks.0." not in k}
    front, est = ck.split_flow_state_dict(gap)
    with pytest.raises(RuntimeError, match="contiguous"):
        ck.flow_shapes(front, est)


def test_fixed_noise_is_the_references_seeded_draw(fcv):
    """``set_all_random_seed(0)`` then ``torch.randn([1, 80, 50 * 300])``
    (flow_matching.py:199-200) on the default CPU generator."""
    with torch.random.fork_rng():
        torch.manual_seed(0)
        ref = torch.randn([1, 80, 50 * 300])
    assert torch.equal(fcv.CFMDecoder(None).rand_noise, ref)
