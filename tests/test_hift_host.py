"""CPU checks of the HiFT boundary: the C struct layout (through the library's weight count),
create-time validation, output lengths, and the strict hift.pt load.  No kernel runs here."""

from __future__ import annotations

import ctypes

import pytest
import torch


def _vocoder(fcv, **kw):
    return fcv.HiFTVocoder(fcv.synthetic.HiFTDims(**kw), device="cpu")


def test_weight_count_reads_the_struct(fcv):
    from faster_cosyvoice_amd import _lib
    v = _vocoder(fcv)
    v._cdims.noise_samples = 1000
    # 2 + 2 + 2S + 2S + 8 D S + 8 D S K + 2 + 10 + 2 + 3 with S = K = D = 3
    assert v._lib.fcv_hift_weight_count(v._cdims) == 321
    bad = _lib.FcvHiftDims.from_buffer_copy(bytes(v._cdims))
    bad.n_fft = 32
    assert v._lib.fcv_hift_weight_count(bad) == 0


def test_create_validates_the_weight_table(fcv):
    from faster_cosyvoice_amd import _lib
    v = _vocoder(fcv)
    v._cdims.noise_samples = 1000
    h = ctypes.c_void_p()
    arr = (ctypes.c_void_p * 321)(*([4096] * 321))
    with pytest.raises(ValueError, match="expected 321"):
        _lib.check(v._lib.fcv_hift_create(v._cdims, arr, 320, h))
    arr[7] = None
    with pytest.raises(ValueError, match="null weight"):
        _lib.check(v._lib.fcv_hift_create(v._cdims, arr, 321, h))
    arr[7] = 4100
    with pytest.raises(ValueError, match="aligned"):
        _lib.check(v._lib.fcv_hift_create(v._cdims, arr, 321, h))


def test_output_lengths_and_short_chunks(fcv):
    from faster_cosyvoice_amd import _lib
    v = _vocoder(fcv)
    v._cdims.noise_samples = 1000
    h = ctypes.c_void_p()
    arr = (ctypes.c_void_p * 321)(*([4096] * 321))
    _lib.check(v._lib.fcv_hift_create(v._cdims, arr, 321, h))
    try:
        lib = v._lib
        assert lib.fcv_hift_output_samples(h, 50, 1) == 50 * 480
        # non-final: 3 frames of F0 lookahead + 4 of conv_pre lookahead + 1 trimmed frame
        assert lib.fcv_hift_output_samples(h, 50, 0) == (50 - 8) * 480
        assert lib.fcv_hift_output_samples(h, 8, 0) == 0
        assert lib.fcv_hift_output_samples(h, 7, 0) == -1
        fr = (ctypes.c_int32 * 1)(2)  # 960 source samples fit the 1000-row noise table
        assert lib.fcv_hift_workspace_bytes(h, fr, None, 1) > 0
        fr[0] = 3  # 1440 source samples exceed the 1000-row noise table
        assert lib.fcv_hift_workspace_bytes(h, fr, None, 1) == 0
    finally:
        v._lib.fcv_hift_destroy(h)


def test_strict_state_dict_load(fcv):
    syn = fcv.synthetic
    dims = syn.HiFTDims()
    v = fcv.HiFTVocoder(dims, device="cpu")
    sd = syn.random_hift_state_dict(dims, seed=0)
    v.load_reference_state_dict({"generator." + k: t for k, t in sd.items()})
    with pytest.raises(RuntimeError, match="missing"):
        v.load_reference_state_dict({k: t for k, t in sd.items() if not k.startswith("conv_post")})
    with pytest.raises(RuntimeError, match="unexpected"):
        v.load_reference_state_dict({**sd, "extra.weight": torch.zeros(1)})
    with pytest.raises(ValueError, match="GPU"):
        v.load_reference_state_dict(sd)
        v.finalize_weights()
