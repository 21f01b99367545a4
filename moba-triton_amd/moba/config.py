"""MoBA configuration: the semantics flags of one attention configuration.

Same fields, defaults and arithmetic as the reference's `MoBAConfig`
(`src/moba/config.py:21-99`), so a config built for the reference means the
same thing here.
"""

import math
from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class MoBAConfig:
    """One MoBA attention configuration (`config.py:21-61`).

    Attributes:
        block_size: Key positions per block.
        top_k: Blocks attended per query; with the defaults this count
            includes the query's own block.
        dtype: Compute dtype of the attention.
        always_select_current: The query's own block is always attended
            (causally masked inside).
        top_k_includes_current: The own block consumes one of the `top_k`
            slots (MoonshotAI's convention). If False it is free.
        tie_break_low_index: Equal gate scores resolve toward the lower block
            index. The HIP gate always resolves this way, which is also a
            valid outcome when the flag is False (the order is then
            unspecified).
        pool_masked_only: Carried for compatibility; the reference's pooling
            averages the whole block regardless (`naive.py:23-61`).
        gate_group: Opt-in hierarchical gate (0, the default, is the exact
            gate): blocks grouped into super-blocks of `gate_group`, whose
            representatives (the mean of their blocks' representatives)
            are gated first; only blocks inside the `gate_open` best
            strictly-past super-blocks and the query's own super-block are
            then ranked. An approximation of the exact selection (the
            reference measured it, `docs/gate-hierarchical-measurements.md`,
            and built no kernel): it changes which blocks are selected.
        gate_open: Super-blocks opened per query when `gate_group` > 0.
    """

    block_size: int
    top_k: int
    dtype: torch.dtype = torch.bfloat16
    always_select_current: bool = True
    top_k_includes_current: bool = True
    tie_break_low_index: bool = True
    pool_masked_only: bool = False
    gate_group: int = 0
    gate_open: int = 0

    def __post_init__(self) -> None:
        if self.block_size <= 0:
            raise ValueError(f"block_size must be positive, got {self.block_size}")
        if self.top_k <= 0:
            raise ValueError(f"top_k must be positive, got {self.top_k}")
        if self.gate_group < 0 or self.gate_open < 0:
            raise ValueError("gate_group and gate_open must be non-negative")
        if self.gate_group > 0 and self.gate_open <= 0:
            raise ValueError("gate_open must be positive when gate_group is set")

    def past_blocks_selected(self, num_blocks: int) -> int:
        """Past-block budget per query, clamped to [0, num_blocks]
        (`config.py:69-84`)."""
        budget = self.top_k
        if self.always_select_current and self.top_k_includes_current:
            budget -= 1
        return max(0, min(budget, num_blocks))

    def num_blocks(self, seq_len: int) -> int:
        """Blocks covering `seq_len` positions, rounded up (`config.py:86-99`)."""
        return math.ceil(seq_len / self.block_size)

    def slots(self) -> int:
        """Most blocks one query can select: the past budget plus the forced
        own block. Equals `top_k` under the default flags, which is the
        reference's `CSCIndex.max_slots` (`routing.py:422`)."""
        budget = self.top_k
        if self.always_select_current and self.top_k_includes_current:
            budget -= 1
        return budget + (1 if self.always_select_current else 0)
