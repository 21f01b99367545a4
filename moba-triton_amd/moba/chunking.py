"""Bounded per-slot buffers (reference `docs/deferred-decisions.md:152-220`, DD-2).

The KV-block-major kernels keep one partial row per (query, slot): `part_acc`
in the forward and the dQ partials in the backward, each top_k times the size
of the output. When those buffers would exceed a budget, the work is split
into chunks of whole (batch row, kv head) units -- heads never interact, and a
kv head's columns carry all of its group's query heads -- and each chunk runs
the unchanged pipeline (pool, gate, CSC, attend, merge; backward likewise)
with buffers sized for the chunk, reused from one chunk to the next. Results
are those of the unchunked run: every stage works per (row, kv head).

A unit whose buffers alone exceed the budget is split further by query head:
a subset of a kv head's query heads is itself a GQA problem over that kv
head. The forward and dQ are those of the unchunked run (every (query, slot)
entry is computed on its own); dK and dV of the kv head are the sum of the
subsets' contributions, added in float32, so they agree with the one-pass
result within rounding rather than bit for bit. The smallest chunk is one
query head of one row.
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


def unit_bytes(tokens: int, group: int, head_dim: int, slots: int, elem: int) -> int:
    """Per-slot buffer bytes of one (batch row, kv head) unit of `tokens`
    tokens (the row's whole token axis; T for packed input): the value rows
    (forward partials, then dQ partials: the larger of the two phases) plus
    the 8-byte (m, l) records.

    Not counted: the CSC index each chunk keeps until backward (12 bytes per
    (query, slot) entry slot, sized sequences x max_seqlen x slots per kv
    head's group when packed). It lives for the whole step whatever the
    chunking, so splitting cannot reduce it."""
    return tokens * group * slots * (head_dim * elem + 8)


def plan_chunks(batch: int, h_kv: int, unit: int, budget: int,
                group: int = 1) -> list[tuple[int, int, int, int, int, int]]:
    """Chunks (b0, b1, hk0, hk1, j0, j1) covering every (batch row, query
    head) once: rows b0..b1, kv heads hk0..hk1 and, of each kv head's `group`
    query heads, those j0..j1 (all of them unless the chunk holds a single
    kv head). Whole batch rows when a row's heads fit together, else kv-head
    groups of one row, else query-head subsets of one unit; each chunk within
    `budget` unless a single query head of one row exceeds it."""
    if batch * h_kv * unit <= budget:
        return [(0, batch, 0, h_kv, 0, group)]
    if h_kv * unit <= budget:
        rows = max(1, budget // (h_kv * unit))
        return [(b0, min(batch, b0 + rows), 0, h_kv, 0, group) for b0 in range(0, batch, rows)]
    if unit <= budget or group == 1:
        heads = max(1, budget // unit)
        return [(b, b + 1, h0, min(h_kv, h0 + heads), 0, group)
                for b in range(batch) for h0 in range(0, h_kv, heads)]
    per = max(1, budget // (unit // group))  # query heads of one unit per chunk
    return [(b, b + 1, hk, hk + 1, j0, min(group, j0 + per))
            for b in range(batch) for hk in range(h_kv) for j0 in range(0, group, per)]


def query_heads(chunk, group: int) -> tuple[int, int]:
    """First and past-the-last query head of a chunk."""
    _, _, hk0, hk1, j0, j1 = chunk
    return hk0 * group + j0, (hk1 - 1) * group + j1


def plan_call(q_shape: tuple, h_kv: int, slots: int, elem: int,
              budget: int) -> list[tuple[int, int, int, int, int, int]]:
    """Chunks of a call on q of shape [B, S, Hq, D] (packed: [1, T, Hq, D]):
    units of one batch row's S tokens per kv head, value rows of `elem`
    bytes."""
    b, s, h_q, d = q_shape
    group = h_q // h_kv
    return plan_chunks(b, h_kv, unit_bytes(s, group, d, slots, elem), budget, group=group)
