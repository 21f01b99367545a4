"""KV-block-major backward (reference `src/moba/kernels/moba_bwd.py`)."""

import torch

from moba import _lib
from moba.config import MoBAConfig
from moba.gqa import head_group_size
from moba.kernels.routing import CSCIndex, index_stride


def compute_delta(out: torch.Tensor, dout: torch.Tensor, lse=None) -> torch.Tensor:
    """delta = rowsum(dO * O), [B, H, S] fp32 (`moba_bwd.py:454-470`).

    With `lse` [B, H, S] given, returns the (lse, delta) pairs [B, H, S, 2]
    the backward kernel reads instead, one 8-byte record per row.
    """
    b, s, h, d = out.shape
    dev = _lib.require_gpu(out, dout)
    out, dout = out.contiguous(), dout.to(out.dtype).contiguous()
    if lse is not None:
        if lse.shape != (b, h, s):
            raise ValueError(f"lse {tuple(lse.shape)} does not match {(b, h, s)}")
        lse = lse.float().contiguous()
    shape = (b, h, s) if lse is None else (b, h, s, 2)
    delta = torch.empty(shape, device=dev, dtype=torch.float32)
    _lib.call("moba_bwd_delta", _lib.ptr(out), _lib.ptr(dout), _lib.ptr(lse),
              _lib.ptr(delta), b, s, h, d, _lib.DTYPE_CODE[out.dtype],
              _lib.stream_handle(dev))
    return delta


def reduce_dq(dq_part: torch.Tensor, part_m: torch.Tensor, out_dtype) -> torch.Tensor:
    """Sums written per-slot dQ partials, [B, S, H, D] (`moba_bwd.py:473-503`)."""
    b, h, s, slots, d = dq_part.shape
    if part_m.shape != (b, h, s, slots):
        raise ValueError(f"part_m {tuple(part_m.shape)} does not match dq_part "
                         f"{tuple(dq_part.shape)}")
    dev = _lib.require_gpu(dq_part, part_m)
    m_stride = 2 if (part_m.dtype == torch.float32 and slots > 0 and
                     part_m.stride() == (2 * h * s * slots, 2 * s * slots, 2 * slots, 2)) else 1
    if m_stride == 1:
        part_m = part_m.float().contiguous()
    dq = torch.empty((b, s, h, d), device=dev, dtype=out_dtype)
    _lib.call("moba_dq_reduce", _lib.ptr(dq_part.contiguous()), _lib.ptr(part_m), m_stride,
              _lib.ptr(dq), b, s, h, d, slots, _lib.DTYPE_CODE[dq_part.dtype],
              _lib.DTYPE_CODE[out_dtype], _lib.stream_handle(dev))
    return dq


def bwd_kernel(dout, q, k, v, lse_delta, cfg: MoBAConfig, index: CSCIndex, dk, dv, dq_part,
               causal: bool = True) -> None:
    """The KV-block-major backward launch (`moba_bwd.py:216-394`): dK, dV
    and one dQ partial per (query, slot), from contiguous q / k / v / dO on
    the GPU and the (lse, delta) pairs of `compute_delta`. dk / dv are in
    q's dtype, or float32 for the unrounded sums."""
    if dk.dtype != dv.dtype or dk.dtype not in (q.dtype, torch.float32):
        raise ValueError(f"dk / dv must both be {q.dtype} or float32, got {dk.dtype}, {dv.dtype}")
    b, s, h_q, d = q.shape
    h_kv = k.shape[2]
    dev = q.device
    rows = index.col_nnz.shape[0]
    mx = index.max_seqlen if index.cu_seqlens is not None else s
    # float32 dK / dV sums of the segments of cut columns
    scratch_cap, scratch = 0, None
    if index.segments is not None and index.seg_cap > index.num_blocks:
        scratch_cap = 2 * (index.seg_cap - index.num_blocks)
        scratch = torch.empty(rows * h_kv * scratch_cap * 2 * cfg.block_size * d,
                              device=dev, dtype=torch.float32)
    _lib.call("moba_bwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(dout),
              _lib.ptr(lse_delta), _lib.ptr(index.col_nnz),
              _lib.ptr(index.col_offsets), _lib.ptr(index.row_indices),
              _lib.ptr(index.head_indices), _lib.ptr(index.slot_of_pair),
              _lib.ptr(index.order), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(dq_part),
              _lib.ptr(index.cu_seqlens), rows, s, mx, h_q, h_kv, d, index.num_blocks,
              cfg.block_size, index.max_slots, index.row_indices.shape[-1], index_stride(index),
              _lib.ptr(index.segments), _lib.ptr(index.seg_split), _lib.ptr(index.seg_counts),
              index.seg_cap, _lib.ptr(scratch), scratch_cap, int(bool(causal)),
              _lib.DTYPE_CODE[q.dtype], _lib.DTYPE_CODE[dq_part.dtype],
              _lib.DTYPE_CODE[dk.dtype], _lib.stream_handle(dev))


def moba_backward(dout, q, k, v, out, lse, part_m, cfg: MoBAConfig, index: CSCIndex,
                  causal: bool = True, dkv_dtype: torch.dtype | None = None):
    """Gradients of the MoBA forward (`moba_bwd.py:506-579`).

    dkv_dtype: None (q's dtype) or torch.float32, for dK / dV sums that the
    caller adds to others (the query-head subsets of one kv head) and
    rounds once.

    Returns:
        (dq, dk, dv) shaped like q, k, v; dk / dv carry H_kv heads, each
        summed over the query heads of its group.
    """
    b, s, h_q, d = q.shape
    h_kv = k.shape[2]
    head_group_size(h_q, h_kv)
    dev = _lib.require_gpu(dout, q, k, v, out, lse, part_m)
    q, k, v = (_lib.aligned_contiguous(t) for t in (q, k, v))
    dout = _lib.aligned_contiguous(dout.to(q.dtype))
    lse_delta = compute_delta(out, dout, lse)
    dk = torch.empty_like(k, dtype=dkv_dtype)
    dv = torch.empty_like(v, dtype=dkv_dtype)
    dq_part = torch.empty((b, h_q, s, index.max_slots, d), device=dev, dtype=q.dtype)
    bwd_kernel(dout, q, k, v, lse_delta, cfg, index, dk, dv, dq_part, causal=causal)
    return reduce_dq(dq_part, part_m, q.dtype), dk, dv
