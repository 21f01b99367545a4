"""Query-head / key-value-head bookkeeping (`src/moba/gqa.py:22-84`).

Query head g reads key/value head g // (H_q // H_kv). The kernels never copy
shared heads: a KV-block column owns its block for every query head of the
group. `expand_kv` exists for callers and tests that want the materialised
form.
"""

import torch


def head_group_size(num_query_heads: int, num_kv_heads: int) -> int:
    """Query heads per key/value head (`gqa.py:22-46`).

    Raises:
        ValueError: If a count is not positive or does not divide.
    """
    if num_query_heads <= 0 or num_kv_heads <= 0:
        raise ValueError(
            f"head counts must be positive, got q={num_query_heads} "
            f"kv={num_kv_heads}")
    if num_query_heads % num_kv_heads != 0:
        raise ValueError(
            f"query heads {num_query_heads} must be divisible by key/value "
            f"heads {num_kv_heads}")
    return num_query_heads // num_kv_heads


def expand_kv(t: torch.Tensor, num_query_heads: int, dim: int = 2) -> torch.Tensor:
    """Repeats each key/value head over its query heads (`gqa.py:49-84`);
    returns `t` itself when the counts already match."""
    group = head_group_size(num_query_heads, t.shape[dim])
    if group == 1:
        return t
    return t.repeat_interleave(group, dim=dim)
