"""KV-block-major backward (reference `src/moba/kernels/moba_bwd.py`)."""

import torch

from moba import _lib
from moba.config import MoBAConfig
from moba.gqa import head_group_size
from moba.kernels.routing import CSCIndex


def compute_delta(out: torch.Tensor, dout: torch.Tensor) -> torch.Tensor:
    """delta = rowsum(dO * O), [B, H, S] fp32 (`moba_bwd.py:454-470`)."""
    b, s, h, d = out.shape
    dev = _lib.require_gpu(out, dout)
    out, dout = out.contiguous(), dout.to(out.dtype).contiguous()
    delta = torch.empty((b, h, s), device=dev, dtype=torch.float32)
    _lib.call("moba_bwd_delta", _lib.ptr(out), _lib.ptr(dout), _lib.ptr(delta),
              b, s, h, d, _lib.DTYPE_CODE[out.dtype], _lib.stream_handle(dev))
    return delta


def reduce_dq(dq_part: torch.Tensor, part_m: torch.Tensor, out_dtype) -> torch.Tensor:
    """Sums written per-slot dQ partials, [B, S, H, D] (`moba_bwd.py:473-503`)."""
    b, h, s, slots, d = dq_part.shape
    if part_m.shape != (b, h, s, slots):
        raise ValueError(f"part_m {tuple(part_m.shape)} does not match dq_part "
                         f"{tuple(dq_part.shape)}")
    dev = _lib.require_gpu(dq_part, part_m)
    dq = torch.empty((b, s, h, d), device=dev, dtype=out_dtype)
    _lib.call("moba_dq_reduce", _lib.ptr(dq_part.contiguous()), _lib.ptr(part_m.contiguous()),
              _lib.ptr(dq), b, s, h, d, slots, _lib.DTYPE_CODE[dq_part.dtype],
              _lib.DTYPE_CODE[out_dtype], _lib.stream_handle(dev))
    return dq


def moba_backward(dout, q, k, v, out, lse, part_m, cfg: MoBAConfig, index: CSCIndex,
                  causal: bool = True):
    """Gradients of the MoBA forward (`moba_bwd.py:506-579`).

    Returns:
        (dq, dk, dv) shaped like q, k, v; dk / dv carry H_kv heads, each
        summed over the query heads of its group.
    """
    b, s, h_q, d = q.shape
    h_kv = k.shape[2]
    head_group_size(h_q, h_kv)
    dev = _lib.require_gpu(dout, q, k, v, out, lse, part_m)
    slots = index.max_slots
    q, k, v = (_lib.aligned_contiguous(t) for t in (q, k, v))
    dout = _lib.aligned_contiguous(dout.to(q.dtype))
    delta = compute_delta(out, dout)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    dq_part = torch.empty((b, h_q, s, slots, d), device=dev, dtype=q.dtype)
    rows = index.col_nnz.shape[0]
    mx = index.max_seqlen if index.cu_seqlens is not None else s
    _lib.call("moba_bwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(dout),
              _lib.ptr(lse.contiguous()), _lib.ptr(delta), _lib.ptr(index.col_nnz),
              _lib.ptr(index.col_offsets), _lib.ptr(index.row_indices),
              _lib.ptr(index.head_indices), _lib.ptr(index.slot_of_pair),
              _lib.ptr(index.order), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(dq_part),
              _lib.ptr(index.cu_seqlens), rows, s, mx, h_q, h_kv, d, index.num_blocks,
              cfg.block_size, slots, index.row_indices.shape[-1], int(bool(causal)),
              _lib.DTYPE_CODE[q.dtype], _lib.DTYPE_CODE[dq_part.dtype],
              _lib.stream_handle(dev))
    return reduce_dq(dq_part, part_m, q.dtype), dk, dv
