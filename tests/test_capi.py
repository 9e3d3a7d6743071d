"""CPU-side checks of the C ABI: the library loads, exports every declared symbol, and its host
validation rejects bad shapes/layouts before touching a GPU; plus host-side helpers."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from oracle import dit_oracle as O

HEADERS = sorted((Path(__file__).resolve().parent.parent / "include").glob("*.h"))


def _declared():
    text = "".join(h.read_text() for h in HEADERS)
    return sorted(set(re.findall(r"\b(fcv_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol(fcv):
    from faster_cosyvoice_amd import _lib
    lib = _lib.load()
    declared = _declared()
    assert declared, "no declarations parsed"
    missing = [name for name in declared if not hasattr(lib, name)]
    assert not missing, missing
    assert set(declared) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"


def test_missing_library_fails_loudly(fcv, monkeypatch, tmp_path):
    """No CPU fallback: without the built HIP library the estimator cannot be used at all."""
    from faster_cosyvoice_amd import _lib
    monkeypatch.setattr(_lib, "_LIB", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libfcvdit.so")
    with pytest.raises(ImportError, match="only compute path"):
        _lib.load()
    # and an estimator never runs on the CPU instead
    est = fcv.DiTEstimator(depth=1, device="cpu")
    with pytest.raises(ValueError, match="GPU device"):
        est.finalize_weights()


def test_struct_layouts(fcv):
    from faster_cosyvoice_amd import _lib
    assert ctypes.sizeof(_lib.FcvDitDims) == 10 * 4
    assert ctypes.sizeof(_lib.FcvDitWeights) == 24 * ctypes.sizeof(ctypes.c_void_p)
    text = "".join(h.read_text() for h in HEADERS)
    body = text[text.index("typedef struct FcvDitWeights"):text.index("} FcvDitWeights;")]
    names = re.findall(r"\*\s*(\w+);", body)
    assert tuple(names) == _lib.WEIGHT_FIELDS
    body = text[text.index("typedef struct FcvFlowDims"):text.index("} FcvFlowDims;")]
    assert tuple(re.findall(r"int32_t\s+(\w+);", body)) == _lib.FLOW_DIM_FIELDS
    body = text[text.index("typedef struct FcvFlowWeights"):text.index("} FcvFlowWeights;")]
    assert tuple(re.findall(r"\*\s*(\w+);", body)) == _lib.FLOW_WEIGHT_FIELDS


def _dims(_lib, **kw):
    base = dict(dim=1024, depth=2, heads=16, dim_head=64, ff_dim=2048, mel_dim=80, conv_kernel=31,
                conv_groups=16, rope_dim=64, max_pos=4096)
    base.update(kw)
    return _lib.FcvDitDims(**base)


def _fake_weights(_lib):
    # host-side validation never dereferences these
    return _lib.FcvDitWeights(**{k: 4096 * (i + 1) for i, k in enumerate(_lib.WEIGHT_FIELDS)})


@pytest.mark.parametrize("bad", [dict(dim=512, heads=8), dict(heads=8), dict(ff_dim=1000),
                                 dict(mel_dim=81), dict(conv_groups=8), dict(conv_kernel=33),
                                 dict(rope_dim=24), dict(depth=0)])
def test_create_rejects_unsupported_dims(fcv, bad):
    from faster_cosyvoice_amd import _lib
    lib = _lib.load()
    handle = ctypes.c_void_p()
    rc = lib.fcv_dit_create(_dims(_lib, **bad), _fake_weights(_lib), handle)
    with pytest.raises(ValueError):
        _lib.check(rc)


def test_create_rejects_null_weight(fcv):
    from faster_cosyvoice_amd import _lib
    lib = _lib.load()
    w = _fake_weights(_lib)
    w.rope_sin = None
    with pytest.raises(ValueError, match="null weight"):
        _lib.check(lib.fcv_dit_create(_dims(_lib), w, ctypes.c_void_p()))


@pytest.fixture()
def handle(fcv):
    from faster_cosyvoice_amd import _lib
    lib = _lib.load()
    h = ctypes.c_void_p()
    _lib.check(lib.fcv_dit_create(_dims(_lib), _fake_weights(_lib), h))
    yield h.value
    lib.fcv_dit_destroy(h.value)


def _plan(_lib, handle, cu, mode=0, chunk=50, ws=1 << 40, nbytes=1 << 40):
    arr = (ctypes.c_int32 * len(cu))(*cu)
    return _lib.load().fcv_dit_plan(handle, arr, len(cu) - 1, mode, chunk, ws, nbytes, None)


@pytest.mark.parametrize("cu,match", [([0], "at least one"), ([1, 5], r"cu_seqlens\[0\]"),
                                      ([0, 5, 5], "length 0"), ([0, 5, 3], "length -2"),
                                      ([0, 5000], "max_pos")])
def test_plan_rejects_bad_layouts(fcv, handle, cu, match):
    from faster_cosyvoice_amd import _lib
    with pytest.raises(ValueError, match=match):
        _lib.check(_plan(_lib, handle, cu))


def test_plan_rejects_layouts_past_32bit_offsets(fcv, handle):
    """128 documents of 4096 rows: (rows + 7 per document) x 4 KB of residual row passes 2 GB,
    past what the kernels' 32-bit buffer ranges address."""
    from faster_cosyvoice_amd import _lib
    cu = [4096 * i for i in range(129)]
    with pytest.raises(ValueError, match="too many rows"):
        _lib.check(_plan(_lib, handle, cu))
    # one document fewer fits the offsets and fails the next check, the workspace size, before
    # anything touches a device
    with pytest.raises(ValueError, match="too small"):
        _lib.check(_plan(_lib, handle, cu[:-1], nbytes=1024))


def test_plan_rejects_bad_mask_and_workspace(fcv, handle):
    from faster_cosyvoice_amd import _lib
    with pytest.raises(ValueError, match="mask_mode"):
        _lib.check(_plan(_lib, handle, [0, 10], mode=7))
    with pytest.raises(ValueError, match="chunk"):
        _lib.check(_plan(_lib, handle, [0, 10], mode=1, chunk=0))
    with pytest.raises(ValueError, match="null workspace"):
        _lib.check(_plan(_lib, handle, [0, 10], ws=0))
    with pytest.raises(ValueError, match="too small"):
        _lib.check(_plan(_lib, handle, [0, 10], nbytes=1024))
    with pytest.raises(ValueError, match="aligned"):
        _lib.check(_plan(_lib, handle, [0, 10], ws=(1 << 40) + 8))


def test_calls_before_plan_raise_state_error(fcv, handle):
    from faster_cosyvoice_amd import _lib
    lib = _lib.load()
    rc = lib.fcv_dit_forward(handle, 1, 1, 1, 1, 1, 1, 1, None)
    with pytest.raises(RuntimeError, match="before fcv_dit_plan"):
        _lib.check(rc)


def test_probe_arm_validates_stage_and_repeat(fcv, handle):
    from faster_cosyvoice_amd import _lib
    lib = _lib.load()
    st = {name: i for i, name in enumerate(_lib.STAGES)}
    with pytest.raises(ValueError, match="unknown stage"):
        _lib.check(lib.fcv_dit_probe_arm(handle, len(_lib.STAGES), 4, 1))
    with pytest.raises(ValueError, match="repeat must be"):
        _lib.check(lib.fcv_dit_probe_arm(handle, st["qkv"], 4, 0))
    # launches that accumulate into their output cannot be repeated inside one event pair
    for name in ("out_proj", "ff2", "euler", "forward"):
        with pytest.raises(ValueError, match="idempotent"):
            _lib.check(lib.fcv_dit_probe_arm(handle, st[name], 4, 2))
    # disarming needs no device
    _lib.check(lib.fcv_dit_probe_arm(handle, st["qkv"], 0, 8))


def test_workspace_bytes_monotone(fcv, handle):
    from faster_cosyvoice_amd import _lib
    lib = _lib.load()
    sizes = [lib.fcv_dit_workspace_bytes(handle, r, n) for r, n in
             [(1, 1), (100, 2), (1000, 2), (1000, 16), (12800, 16), (138000, 128)]]
    assert all(a <= b for a, b in zip(sizes, sizes[1:]))
    assert sizes[-1] < 8 << 30


# ---- host helpers ---------------------------------------------------------------------------


def test_euler_schedule_matches_reference_recurrence(fcv):
    ts, dts = fcv.euler_schedule(10)
    span = O.cosine_schedule(10)
    assert ts[0] == 0.0 and len(ts) == len(dts) == 10
    for k in range(10):
        assert abs(ts[k] - float(span[k])) < 1e-6
        assert abs(ts[k] + dts[k] - float(span[k + 1])) < 1e-6


def test_rope_tables_match_oracle_angles(fcv):
    cos, sin = fcv.rope_tables(300, 64, 64)
    freqs = O.rotary_freqs(torch.arange(300), 64)[:, 0::2]
    torch.testing.assert_close(cos, freqs.cos())
    torch.testing.assert_close(sin, freqs.sin())


def test_flop_count_per_row(fcv):
    f = fcv.synthetic.flops_per_forward([1], streaming=False)
    assert abs(f["dense"] - 378.04e6) < 0.01e6
    assert f["attention"] == 4 * 16 * 64 * 22
    g = fcv.synthetic.flops_per_forward([120], streaming=True, chunk=50)
    # chunk-causal visible pairs: 50 rows see 50, 50 see 100, 20 see 120
    assert g["pairs"] == 50 * 50 + 50 * 100 + 20 * 120


@pytest.mark.parametrize("index", [1, 2, 3, 4, 5])
def test_workloads(fcv, index):
    b = fcv.synthetic.workload(index)
    assert b.noise.shape == (sum(b.lengths), 80) and b.spks.shape == (len(b.lengths), 80)
    assert all(0 <= p <= n for p, n in zip(b.prompt_lengths, b.lengths))
    expect_req = {1: 1, 2: 1, 3: 8, 4: 32, 5: 64}[index]
    assert b.n_requests == expect_req
    if index == 3:
        assert all(100 <= n <= 1500 for n in b.lengths)
    if index == 4:
        assert b.streaming and all(h in (30, 60, 120) for h in b.meta["hops"])
    if index == 5:
        assert all(64 <= n <= 3000 for n in b.lengths)
    # cond holds the prompt frames only
    off = 0
    for n, p in zip(b.lengths, b.prompt_lengths):
        assert torch.all(b.cond[off + p:off + n] == 0)
        off += n
