"""Stage 1: block representatives (reference `src/moba/kernels/pooling.py`)."""

import torch

from moba import _lib
from moba.config import MoBAConfig
from moba.varlen import validate_cu_seqlens


def pool_blocks(k: torch.Tensor, cfg: MoBAConfig,
                cu_seqlens: torch.Tensor | None = None,
                max_seqlen: int | None = None) -> torch.Tensor:
    """Mean-pools each block's keys (`pooling.py:103-163`).

    Args:
        k: Keys [B, S, H, D] (or [1, T, H, D] packed), on the GPU.
        cfg: Supplies `block_size`.
        cu_seqlens: int32 [n_seq + 1] when packed.
        max_seqlen: Longest sequence; required with `cu_seqlens`.

    Returns:
        kbar, k.dtype: [B, H, nb, D], or [n_seq, H, cdiv(max_seqlen, bs), D]
        packed (rows past a sequence's own block count are left unwritten).
    """
    b, s, h, d = k.shape
    dev = _lib.require_gpu(k, cu_seqlens)
    k = _lib.aligned_contiguous(k)
    if cu_seqlens is None:
        rows, n, mx = b, cfg.num_blocks(s), s
    else:
        if b != 1:
            raise ValueError(f"packed input must have batch 1, got {b}")
        if max_seqlen is None:
            raise ValueError("max_seqlen is required when cu_seqlens is given")
        rows = validate_cu_seqlens(cu_seqlens, total_tokens=s, max_seqlen=max_seqlen)
        n, mx = cfg.num_blocks(max_seqlen), max_seqlen
    out = torch.empty((rows, h, n, d), device=dev, dtype=k.dtype)
    _lib.call("moba_pool", _lib.ptr(k), _lib.ptr(out), _lib.ptr(cu_seqlens),
              rows, s, mx, h, d, n, cfg.block_size, _lib.DTYPE_CODE[k.dtype],
              _lib.stream_handle(dev))
    return out
