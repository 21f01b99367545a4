"""Stage 2: the gate (reference `src/moba/kernels/gating.py`)."""

import torch

from moba import _lib
from moba.config import MoBAConfig
from moba.gqa import head_group_size
from moba.varlen import validate_cu_seqlens


def gate_select(q: torch.Tensor, kbar: torch.Tensor, cfg: MoBAConfig,
                cu_seqlens: torch.Tensor | None = None,
                max_seqlen: int | None = None) -> torch.Tensor:
    """Selected block ids per query (`gating.py:343-448`).

    Returns:
        int32 [B, H, S, slots], ascending per query, -1 padded; ids are
        sequence-local when packed. `slots` is `cfg.slots()` (= top_k under
        the default flags).

    Raises:
        ValueError: On shape / head-count / packing errors.
    """
    b, s, h, d = q.shape
    dev = _lib.require_gpu(q, kbar, cu_seqlens)
    if cu_seqlens is not None:
        if b != 1:
            raise ValueError(f"packed input must have batch 1, got {b}")
        if max_seqlen is None:
            raise ValueError("max_seqlen is required when cu_seqlens is given")
        rows = validate_cu_seqlens(cu_seqlens, total_tokens=s, max_seqlen=max_seqlen)
        take = cfg.past_blocks_selected(cfg.num_blocks(max_seqlen))
        mx = max_seqlen
    else:
        rows, mx = b, s
        take = cfg.past_blocks_selected(kbar.shape[2])
    if kbar.shape[0] != rows or kbar.shape[-1] != d:
        raise ValueError(f"representative shape {tuple(kbar.shape)} does not match "
                         f"queries {tuple(q.shape)}")
    head_group_size(h, kbar.shape[1])
    q = _lib.aligned_contiguous(q)
    kbar = _lib.aligned_contiguous(kbar)
    slots = cfg.slots()
    out = torch.empty((b, h, s, slots), device=dev, dtype=torch.int32)
    ws_bytes = _lib.load().moba_gate_workspace_size(rows, mx if cu_seqlens is not None else s, h)
    ws = torch.empty(max(int(ws_bytes), 256), device=dev, dtype=torch.uint8)
    _lib.call("moba_gate", _lib.ptr(q), _lib.ptr(kbar), _lib.ptr(out),
              _lib.ptr(cu_seqlens), rows, s, mx, h, kbar.shape[1], d, kbar.shape[2],
              cfg.block_size, slots, take, int(bool(cfg.always_select_current)),
              _lib.DTYPE_CODE[q.dtype], _lib.ptr(ws), ws.numel(), _lib.stream_handle(dev))
    return out
