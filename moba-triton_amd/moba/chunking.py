"""Bounded per-slot buffers (reference `docs/deferred-decisions.md:152-220`, DD-2).

The KV-block-major kernels keep one partial row per (query, slot): `part_acc`
in the forward and the dQ partials in the backward, each top_k times the size
of the output. When those buffers would exceed a budget, the work is split
into chunks of whole (batch row, kv head) units -- heads never interact, and a
kv head's columns carry all of its group's query heads -- and each chunk runs
the unchanged pipeline (pool, gate, CSC, attend, merge; backward likewise)
with buffers sized for the chunk, reused from one chunk to the next. Results
are those of the unchunked run: every stage works per (row, kv head).

A single (row, kv head) unit is never split (that would need query chunks),
so the smallest chunk's buffers are one unit's.
"""

import os

import torch

ENV_BUDGET = "MOBA_PARTIALS_BUDGET_BYTES"


def partials_budget(device) -> int:
    """Bytes the per-slot buffers may take: `MOBA_PARTIALS_BUDGET_BYTES` when
    set, else a quarter of the device's memory or half of what is free now,
    whichever is smaller."""
    env = os.environ.get(ENV_BUDGET)
    if env:
        return int(env)
    free, total = torch.cuda.mem_get_info(device)
    return min(total // 4, free // 2)


def unit_bytes(rows_per_seq: int, group: int, head_dim: int, slots: int, elem: int) -> int:
    """Per-slot buffer bytes of one (batch row, kv head) unit: the value rows
    (forward partials, then dQ partials: the larger of the two phases) plus
    the 8-byte (m, l) records."""
    return rows_per_seq * group * slots * (head_dim * elem + 8)


def plan_chunks(batch: int, h_kv: int, unit: int, budget: int) -> list[tuple[int, int, int, int]]:
    """Chunks (b0, b1, hk0, hk1) covering every (batch row, kv head) once:
    whole batch rows when a row's heads fit together, else head groups of
    one row; each chunk within `budget` unless a single unit exceeds it."""
    if batch * h_kv * unit <= budget:
        return [(0, batch, 0, h_kv)]
    if h_kv * unit <= budget:
        rows = max(1, budget // (h_kv * unit))
        return [(b0, min(batch, b0 + rows), 0, h_kv) for b0 in range(0, batch, rows)]
    heads = max(1, budget // unit)
    return [(b, b + 1, h0, min(h_kv, h0 + heads))
            for b in range(batch) for h0 in range(0, h_kv, heads)]
