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
    if cfg.gate_group > 0:
        if cu_seqlens is not None:
            raise ValueError("the hierarchical gate (gate_group > 0) takes padded input only")
        return hierarchical_select(q, kbar, cfg)
    slots = cfg.slots()
    out = torch.empty((b, h, s, slots), device=dev, dtype=torch.int32)
    ws_bytes = _lib.load().moba_gate_workspace_size(rows, mx if cu_seqlens is not None else s, h)
    ws = torch.empty(max(int(ws_bytes), 256), device=dev, dtype=torch.uint8)
    _lib.call("moba_gate", _lib.ptr(q), _lib.ptr(kbar), _lib.ptr(out),
              _lib.ptr(cu_seqlens), rows, s, mx, h, kbar.shape[1], d, kbar.shape[2],
              cfg.block_size, slots, take, int(bool(cfg.always_select_current)),
              _lib.DTYPE_CODE[q.dtype], _lib.ptr(ws), ws.numel(), _lib.stream_handle(dev))
    return out


def super_block_means(kbar: torch.Tensor, group: int) -> torch.Tensor:
    """Super-block representatives [B, H, cdiv(nb, group), D]: the block
    representatives pooled `group` at a time by the pool kernel, which sees
    kbar [B, H, nb, D] as B * H rows of nb one-head 'keys'."""
    b, h, n, d = kbar.shape
    dev = _lib.require_gpu(kbar)
    kbar = _lib.aligned_contiguous(kbar)
    nsb = -(-n // group)
    out = torch.empty((b, h, nsb, d), device=dev, dtype=kbar.dtype)
    _lib.call("moba_pool", _lib.ptr(kbar), _lib.ptr(out), None, b * h, n, n, 1, d, nsb, group,
              _lib.DTYPE_CODE[kbar.dtype], _lib.stream_handle(dev))
    return out


def hierarchical_select(q: torch.Tensor, kbar: torch.Tensor, cfg: MoBAConfig) -> torch.Tensor:
    """The opt-in coarse-to-fine gate (`cfg.gate_group` > 0; reference
    `docs/gate-hierarchical-measurements.md`): the exact gate over
    super-block representatives opens `cfg.gate_open` strictly-past
    super-blocks plus the query's own, then `moba_gate_refine` ranks the
    strictly-past blocks inside them. Same output contract as the exact
    gate: int32 [B, H, S, slots], ascending, -1 padded."""
    b, s, h, d = q.shape
    dev = q.device
    group, n = cfg.gate_group, kbar.shape[2]
    sbar = super_block_means(kbar, group)
    nsb = sbar.shape[2]
    sup_take = min(cfg.gate_open, nsb)
    sup = torch.empty((b, h, s, cfg.gate_open + 1), device=dev, dtype=torch.int32)
    lib = _lib.load()
    ws = torch.empty(max(int(lib.moba_gate_workspace_size(b, s, h)), 256), device=dev,
                     dtype=torch.uint8)
    stream = _lib.stream_handle(dev)
    _lib.call("moba_gate", _lib.ptr(q), _lib.ptr(sbar), _lib.ptr(sup), None, b, s, s, h,
              kbar.shape[1], d, nsb, cfg.block_size * group, cfg.gate_open + 1, sup_take, 1,
              _lib.DTYPE_CODE[q.dtype], _lib.ptr(ws), ws.numel(), stream)
    slots = cfg.slots()
    out = torch.empty((b, h, s, slots), device=dev, dtype=torch.int32)
    _lib.call("moba_gate_refine", _lib.ptr(q), _lib.ptr(kbar), _lib.ptr(sup), _lib.ptr(out), b,
              s, h, kbar.shape[1], d, n, cfg.block_size, group, cfg.gate_open + 1, slots,
              cfg.past_blocks_selected(n), int(bool(cfg.always_select_current)),
              _lib.DTYPE_CODE[q.dtype], stream)
    return out
