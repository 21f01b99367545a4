"""The varlen MoBA signature of ReyJerry/Triton-MoBA, served by the HIP
kernels (reference adapter `implementations/triton_moba.py:72-84`).

`moba_attn_varlen_triton(q, k, v, cu_seqlens, max_seqlen, moba_chunk_size,
moba_topk)` takes packed `[T, H, D]` tensors and returns `[T, H, D]`. Its
`moba_topk` counts the query's own block (MoonshotAI's convention, which is
`MoBAConfig`'s default `top_k_includes_current=True`). Differentiable.

Only the signature lives here. The reference registers "triton_moba" as a
vendored third-party backend (`implementations/triton_moba.py:32-36`); this
build registers nothing under that name, so a harness comparing backends never
reports these kernels as a second implementation.
"""

import torch

from moba.config import MoBAConfig
from moba.kernels.attention import moba_attention


def moba_attn_varlen_triton(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                            cu_seqlens: torch.Tensor, max_seqlen: int,
                            moba_chunk_size: int, moba_topk: int) -> torch.Tensor:
    """Packed MoBA attention: q [T, Hq, D], k / v [T, Hkv, D], cu_seqlens
    [n + 1] (any integer dtype), returns [T, Hq, D]."""
    if q.ndim != 3:
        raise ValueError(f"expected packed [T, H, D] queries, got {tuple(q.shape)}")
    cfg = MoBAConfig(block_size=int(moba_chunk_size), top_k=int(moba_topk), dtype=q.dtype)
    out = moba_attention(q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0), cfg,
                         cu_seqlens=cu_seqlens.to(torch.int32), max_seqlen=int(max_seqlen))
    return out.squeeze(0)


# Name kept by the reference adapter's caller.
moba_attn_varlen = moba_attn_varlen_triton
