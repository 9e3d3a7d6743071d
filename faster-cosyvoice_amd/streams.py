"""Process-wide streams for concurrent request groups.

A process gets a few hardware queues per GPU (four by default on ROCm); streams beyond those
share queues, and the work of two streams on one queue runs one after the other.  So every
component that runs request groups concurrently (the DiT solver, the HiFT vocoder) takes
group ``i``'s stream from this one pool: the process then uses the default stream plus one
stream per group, whatever is built.  Group work is launched from one thread, like the
reference's single token2wav executor, so sharing the streams orders nothing that would
otherwise overlap.  All streams have the default priority.
"""

from __future__ import annotations

import torch

_POOL: dict[tuple[int, int], torch.cuda.Stream] = {}


def group_stream(device: torch.device | str, group: int) -> torch.cuda.Stream:
    """The stream request group ``group`` runs on, on ``device`` (created on first use)."""
    dev = torch.device(device)
    index = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (index, int(group))
    if key not in _POOL:
        _POOL[key] = torch.cuda.Stream(device=torch.device("cuda", index))
    return _POOL[key]
