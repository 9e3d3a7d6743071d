"""MI355X-native (gfx950) CosyVoice3 Token2Wav DiT estimator: packed CFG batches, hand-written
HIP kernels behind the C ABI of libfcvdit.so (include/fcv_dit.h).

Public surface (mirrors faster_cosyvoice.token2wav.flashinfer_dit / flashinfer_flow):
  DiTEstimator            -- the estimator plugin (FlashInferDiT counterpart)
  solve_euler_packed      -- packed CFG Euler solve, optionally one hipGraph
  solve_euler_batched     -- padded drop-in of the reference solver
  apply_mi355x            -- install into a Token2Wav flow (apply_flashinfer counterpart)
  FlowFrontEnd            -- tokens / prompt Mel / x-vectors -> packed mu, cond, spks
  flow_inference_batched, flow_inference_batched_streaming
                          -- the flow entry points, front-end through packed solve
  StreamingFlow, CFMDecoder
                          -- stream_step / stream_step_batched (Flow half) over the packed path
  load_flow               -- the MI355X flow from a flow.pt state dict
  HiFTVocoder             -- the HiFT vocoder (CausalHiFTGenerator counterpart), packed batches
"""

from .estimator import DiTEstimator, rope_tables
from .frontend import FlowFrontEnd, flow_inference_batched, flow_inference_batched_streaming
from .solver import apply_mi355x, euler_schedule, solve_euler_batched, solve_euler_packed
from .streaming import CFMDecoder, StreamingFlow
from .checkpoint import load_flow
from .hift import HiFTVocoder
from . import synthetic

__all__ = ["CFMDecoder", "DiTEstimator", "FlowFrontEnd", "HiFTVocoder", "StreamingFlow",
           "apply_mi355x",
           "euler_schedule",
           "flow_inference_batched", "flow_inference_batched_streaming", "load_flow", "rope_tables",
           "solve_euler_batched", "solve_euler_packed", "synthetic"]
