"""Loading helpers for the fixtures in tests/golden/ (written by tests/golden/make_golden.py)."""
import hashlib
import os

import numpy as np
import torch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def digest(t: torch.Tensor) -> str:
    t = t.contiguous()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return hashlib.sha256(t.numpy().tobytes()).hexdigest()


def from_bits(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)


def events_array(events, width):
    """Event dicts -> the [m, 4 + width] int32 layout of the fixture."""
    ev = np.full((len(events), 4 + width), -1, dtype=np.int32)
    for i, e in enumerate(events):
        f = e["freed_block_ids"]
        ev[i, :4] = [e["batch_index"], e["new_context_len"], e["keep_blocks"], len(f)]
        ev[i, 4:4 + len(f)] = f
    return ev
