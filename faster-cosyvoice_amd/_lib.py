"""ctypes bindings of libfcvdit.so (declared in include/fcv_dit.h, fcv_flow.h and fcv_hift.h).

The library is the only compute path: if it is missing, importing the estimator raises,
there is no fallback.  Error codes map to the exceptions the reference raises for the same
conditions (flashinfer_dit.py:326-327 ValueError for bad inputs, :235-236 and :979-983
RuntimeError for state errors).
"""

from __future__ import annotations

import ctypes
from ctypes import POINTER, c_float, c_int32, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libfcvdit.so"

FCV_OK, FCV_ERR_INVALID, FCV_ERR_RUNTIME, FCV_ERR_STATE = 0, 1, 2, 3
FCV_MASK_FULL, FCV_MASK_CHUNK_CAUSAL = 0, 1

DIM_FIELDS = ("dim", "depth", "heads", "dim_head", "ff_dim", "mel_dim", "conv_kernel",
              "conv_groups", "rope_dim", "max_pos")

WEIGHT_FIELDS = (
    "temb_w1", "temb_b1", "temb_w2", "temb_b2", "ada_w", "ada_b", "in_w", "in_b",
    "conv1_w", "conv1_b", "conv2_w", "conv2_b", "qkv_w", "qkv_b", "out_w", "out_b",
    "ff1_w", "ff1_b", "ff2_w", "ff2_b", "proj_w", "proj_b", "rope_cos", "rope_sin",
)


class FcvDitDims(ctypes.Structure):
    _fields_ = [(name, c_int32) for name in DIM_FIELDS]


class FcvDitWeights(ctypes.Structure):
    _fields_ = [(name, c_void_p) for name in WEIGHT_FIELDS]


FLOW_MAX_DOCS = 256  # FCV_FLOW_MAX_DOCS
FLOW_DIM_FIELDS = ("vocab", "feat_dim", "channels", "lookahead", "token_mel_ratio", "spk_dim")
FLOW_WEIGHT_FIELDS = ("embed", "la1_w", "la1_b", "la2_w", "la2_b", "spk_w", "spk_b")


class FcvFlowDims(ctypes.Structure):
    _fields_ = [(name, c_int32) for name in FLOW_DIM_FIELDS]


class FcvFlowWeights(ctypes.Structure):
    _fields_ = [(name, c_void_p) for name in FLOW_WEIGHT_FIELDS]


HIFT_MAX = 4          # FCV_HIFT_MAX
HIFT_MAX_DOCS = 256   # FCV_HIFT_MAX_DOCS
_I4 = c_int32 * HIFT_MAX


class FcvHiftDims(ctypes.Structure):
    _fields_ = [
        ("in_channels", c_int32), ("base_channels", c_int32), ("nb_harmonics", c_int32),
        ("sampling_rate", c_int32), ("nsf_alpha", c_float), ("nsf_sigma", c_float),
        ("nsf_voiced_threshold", c_float), ("n_stages", c_int32), ("upsample_rates", _I4),
        ("upsample_kernels", _I4), ("n_kernels", c_int32), ("resblock_kernels", _I4),
        ("n_dilations", c_int32), ("resblock_dilations", _I4 * HIFT_MAX),
        ("source_kernels", _I4), ("source_dilations", _I4 * HIFT_MAX), ("n_fft", c_int32),
        ("hop_len", c_int32), ("conv_pre_look_right", c_int32), ("f0_channels", c_int32),
        ("lrelu_slope", c_float), ("audio_limit", c_float), ("noise_samples", c_int32),
    ]


# (name, restype, argtypes) of every exported entry point
SIGNATURES = {
    "fcv_last_error": (ctypes.c_char_p, []),
    "fcv_dit_create": (c_int32, [POINTER(FcvDitDims), POINTER(FcvDitWeights), POINTER(c_void_p)]),
    "fcv_dit_destroy": (c_int32, [c_void_p]),
    "fcv_dit_workspace_bytes": (c_size_t, [c_void_p, c_int32, c_int32]),
    "fcv_dit_plan": (c_int32, [c_void_p, POINTER(c_int32), c_int32, c_int32, c_int32, c_void_p,
                               c_size_t, c_void_p]),
    "fcv_dit_plan_capacity": (c_int32, [c_void_p, POINTER(c_int32), c_int32, c_int32, c_int32,
                                        c_int32, c_int32, c_void_p, c_size_t, c_void_p]),
    "fcv_dit_graph_stats": (c_int32, [c_void_p, POINTER(c_int32), POINTER(c_int32)]),
    "fcv_dit_plan_info": (c_int32, [c_void_p, POINTER(c_int32), POINTER(c_int32),
                                    POINTER(c_int32)]),
    "fcv_dit_forward": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                  c_int32, c_void_p, c_void_p]),
    "fcv_euler_cfg_step": (c_int32, [c_void_p, c_void_p, c_void_p, c_float, c_float, c_void_p]),
    "fcv_dit_solve": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                POINTER(c_float), POINTER(c_float), c_int32, c_float, c_int32,
                                c_void_p]),
    "fcv_dit_schedule_bytes": (c_size_t, [c_void_p, c_int32]),
    "fcv_dit_schedule": (c_int32, [c_void_p, POINTER(c_float), c_int32, c_void_p, c_size_t,
                                   c_void_p]),
    "fcv_dit_solve_scheduled": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                          POINTER(c_float), c_int32, c_float, c_void_p,
                                          c_size_t, c_int32, c_void_p]),
    "fcv_pack_padded": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p,
                                  c_void_p]),
    "fcv_unpack_padded": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p,
                                    c_void_p]),
    "fcv_dit_probe_arm": (c_int32, [c_void_p, c_int32, c_int32, c_int32]),
    "fcv_dit_probe_read": (c_int32, [c_void_p, POINTER(c_float), c_int32, POINTER(c_int32)]),
    # include/fcv_flow.h
    "fcv_flow_workspace_bytes": (c_size_t, [POINTER(FcvFlowDims), c_int32]),
    "fcv_flow_token_features": (c_int32, [POINTER(FcvFlowDims), POINTER(FcvFlowWeights), c_void_p,
                                          POINTER(c_int32), POINTER(c_int32), c_int32, c_void_p,
                                          c_void_p, c_size_t, c_void_p]),
    "fcv_flow_token_features_noalloc": (c_int32, [POINTER(FcvFlowDims), POINTER(FcvFlowWeights),
                                                  c_void_p, POINTER(c_int32), POINTER(c_int32),
                                                  c_int32, c_void_p, c_void_p]),
    "fcv_flow_speaker": (c_int32, [POINTER(FcvFlowDims), POINTER(FcvFlowWeights), c_void_p,
                                   c_int32, c_void_p, c_void_p]),
    "fcv_flow_prompt_cond": (c_int32, [POINTER(FcvFlowDims), c_void_p, POINTER(c_int32),
                                       POINTER(c_int32), c_int32, c_void_p, c_void_p]),
    # include/fcv_hift.h
    "fcv_hift_weight_count": (c_int32, [POINTER(FcvHiftDims)]),
    "fcv_hift_create": (c_int32, [POINTER(FcvHiftDims), POINTER(c_void_p), c_int32,
                                  POINTER(c_void_p)]),
    "fcv_hift_destroy": (c_int32, [c_void_p]),
    "fcv_hift_output_samples": (ctypes.c_int64, [c_void_p, c_int32, c_int32]),
    "fcv_hift_workspace_bytes": (c_size_t, [c_void_p, POINTER(c_int32), POINTER(c_int32),
                                            c_int32]),
    "fcv_hift_inference": (c_int32, [c_void_p, c_void_p, POINTER(c_int32), POINTER(c_int32),
                                     c_int32, c_void_p, c_void_p, c_void_p, c_size_t,
                                     c_void_p]),
    "fcv_hift_workspace_bytes_capacity": (c_size_t, [c_void_p, c_int32, c_int32]),
    "fcv_hift_inference_capacity": (c_int32, [c_void_p, c_void_p, POINTER(c_int32),
                                              POINTER(c_int32), c_int32, c_int32, c_int32,
                                              c_void_p, c_void_p, c_void_p, c_size_t, c_int32,
                                              c_void_p]),
    "fcv_hift_graph_stats": (c_int32, [c_void_p, POINTER(c_int32), POINTER(c_int32)]),
}

STAGES = ("qkv", "attention", "out_proj", "ff1", "ff2", "ln_mod", "conv", "adaln", "in_proj",
          "proj_out", "euler", "forward")

_LIB: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load libfcvdit.so once; raise ImportError when it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH} is missing: build it with `python faster-cosyvoice_amd/build.py` "
                          "(the HIP library is the only compute path)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _LIB = lib
    return lib


def check(rc: int) -> None:
    """Raise the Python exception that matches a library status code."""
    if rc == FCV_OK:
        return
    msg = load().fcv_last_error().decode(errors="replace")
    if rc == FCV_ERR_INVALID:
        raise ValueError(msg)
    raise RuntimeError(msg)
