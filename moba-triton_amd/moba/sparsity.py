"""Closed-form sparsity of the MoBA pattern (reference `bench/suite.py:66-95`).

The fraction of causally legal keys a query attends to, over a whole
sequence: query i keeps the visible prefix of its own block, i - own*bs + 1
keys, plus every key of min(own, past budget) selected past blocks. The
attainment ceiling of a benchmark row is its inverse.
"""

import torch

from moba.config import MoBAConfig


def sparsity_ratio(seq_len: int, cfg: MoBAConfig) -> float:
    """Attended keys over causally legal keys, in (0, 1]; 1.0 is dense."""
    bs = cfg.block_size
    past = cfg.past_blocks_selected(cfg.num_blocks(seq_len))
    i = torch.arange(seq_len, dtype=torch.float64)
    own = torch.div(i, bs, rounding_mode="floor")
    attended = (i - own * bs + 1) + torch.clamp(own, max=float(past)) * bs
    return (attended.sum() / (i + 1).sum()).item()
