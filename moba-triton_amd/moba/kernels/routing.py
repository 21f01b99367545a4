"""Stage 3: the CSC transpose (reference `src/moba/kernels/routing.py`)."""

from dataclasses import dataclass

import os

import torch

from moba import _lib
from moba.config import MoBAConfig
from moba.gqa import head_group_size
from moba.kernels.gating import gate_select
from moba.kernels.pooling import pool_blocks
from moba.varlen import validate_cu_seqlens


@dataclass(frozen=True)
class CSCIndex:
    """KV-block-major view of the routing decision (`routing.py:73-130`).

    Attributes:
        col_nnz: Queries selecting each block, [R, H_kv, nb] int32.
        col_offsets: Exclusive prefix sum of `col_nnz`, [R, H_kv, nb + 1].
        row_indices: Query positions grouped by block, [R, H_kv, cap] int32,
            cap = (H_q / H_kv) * rows_per_seq * slots; entries past a
            column's extent are undefined, order inside a column is
            unspecified (atomic cursor). Packed: packed token indices.
        head_indices: Query head of each entry, aligned with `row_indices`.
        slot_of_pair: The query's output slot each entry fills.
        order: Column ids by count desc, id asc (longest first).
        num_blocks: Blocks per (padded) sequence.
        max_slots: Partial slots reserved per query (`cfg.slots()`).
        num_query_heads: H_q.
        cu_seqlens / max_seqlen: Packing metadata, None when padded.
    """

    col_nnz: torch.Tensor
    col_offsets: torch.Tensor
    row_indices: torch.Tensor
    head_indices: torch.Tensor
    slot_of_pair: torch.Tensor
    order: torch.Tensor
    num_blocks: int
    max_slots: int
    num_query_heads: int
    cu_seqlens: torch.Tensor | None = None
    max_seqlen: int | None = None
    # Segment list (this build's addition; None: one program per column).
    segments: torch.Tensor | None = None     # [R, H_kv, seg_cap, 4] int32
    seg_split: torch.Tensor | None = None    # [R, H_kv, seg_cap - nb] int32
    seg_counts: torch.Tensor | None = None   # [R, H_kv, 2] int32
    seg_cap: int = 0


ENV_SEGMENT = "MOBA_SEGMENT_ENTRIES"
MAX_SEGMENTS = 8


def segment_entries(total_pairs: int) -> int:
    """Longest column segment one program takes: half of one workgroup
    slot's share of all (query, slot) pairs (about 1024 programs run at
    once), at least 2048 -- so only columns that would outlast the other
    programs are cut (none at S = 512K, the longest few at 64K).
    `MOBA_SEGMENT_ENTRIES` overrides it; 0 turns cutting off."""
    env = os.environ.get(ENV_SEGMENT)
    if env is not None:
        return int(env)
    return max(2048, -(-total_pairs // 1024))


def index_stride(index: CSCIndex) -> int:
    """Element stride shared by the three index arrays (3 for the record
    layout `build_csc_from_indices` makes, 1 for separate arrays).

    Raises:
        ValueError: If the arrays differ in dtype, shape or strides, or are
            not uniformly strided over (row, kv head, entry).
    """
    fields = (index.row_indices, index.head_indices, index.slot_of_pair)
    if any(t.dtype != torch.int32 for t in fields):
        raise ValueError("index arrays must be int32")
    if len({tuple(t.shape) for t in fields}) != 1 or len({t.stride() for t in fields}) != 1:
        raise ValueError("row_indices, head_indices and slot_of_pair must share shape and strides")
    shape, st = fields[0].shape, fields[0].stride()
    step = st[-1]
    run = step
    for n, s_ in zip(reversed(shape), reversed(st)):
        if n != 1 and s_ != run:
            raise ValueError("index arrays must be uniformly strided over (row, kv head, entry)")
        run *= n
    return int(step)


def build_csc_from_indices(block_idx: torch.Tensor, num_blocks: int, cfg: MoBAConfig,
                           num_kv_heads: int | None = None,
                           cu_seqlens: torch.Tensor | None = None,
                           max_seqlen: int | None = None) -> CSCIndex:
    """Transposes per-query ids into a CSC index (`routing.py:309-427`).

    Args:
        block_idx: int32 [B, H_q, S, slots], -1 padded, as `gate_select`
            returns.
        num_blocks: Columns per (padded) sequence.
        cfg: Configuration.
        num_kv_heads: H_kv (defaults to H_q).
        cu_seqlens / max_seqlen: Packing metadata.
    """
    b, h_q, s, slots = block_idx.shape
    h_kv = h_q if num_kv_heads is None else num_kv_heads
    group = head_group_size(h_q, h_kv)
    dev = _lib.require_gpu(block_idx, cu_seqlens)
    if cu_seqlens is not None:
        if b != 1:
            raise ValueError(f"packed block ids must have batch 1, got {b}")
        if max_seqlen is None:
            raise ValueError("max_seqlen is required when cu_seqlens is given")
        rows = validate_cu_seqlens(cu_seqlens, total_tokens=s, max_seqlen=max_seqlen)
        rps = max_seqlen
    else:
        rows, rps = b, s
    cap = group * rps * slots
    block_idx = block_idx.contiguous()
    i32 = dict(device=dev, dtype=torch.int32)
    col_nnz = torch.empty(rows, h_kv, num_blocks, **i32)
    col_offsets = torch.empty(rows, h_kv, num_blocks + 1, **i32)
    order = torch.empty(rows, h_kv, num_blocks, **i32)
    # One (row, head, slot) record per entry: the scatter writes each entry
    # into one memory sector. The three fields are strided views of it.
    entries = torch.empty(rows, h_kv, cap, 3, **i32)
    row_indices, head_indices, slot_of_pair = entries.unbind(-1)
    seg_len = segment_entries(rows * h_q * rps * slots)
    seg = split = counts = None
    seg_cap = 0
    if seg_len > 0:
        seg_cap = num_blocks + -(-(group * rps * slots) // seg_len)
        seg = torch.empty(rows, h_kv, seg_cap, 4, **i32)
        split = torch.empty(rows, h_kv, seg_cap - num_blocks, **i32)
        counts = torch.empty(rows, h_kv, 2, **i32)
    lib = _lib.load()
    ws_bytes = int(lib.moba_csc_workspace_size(rows, rps, h_q, h_kv, num_blocks, slots))
    ws = torch.empty(max(ws_bytes, 256), device=dev, dtype=torch.uint8)
    _lib.call("moba_csc_build", _lib.ptr(block_idx), _lib.ptr(col_nnz),
              _lib.ptr(col_offsets), _lib.ptr(row_indices), _lib.ptr(head_indices),
              _lib.ptr(slot_of_pair), _lib.ptr(order), _lib.ptr(cu_seqlens), rows, s,
              rps, h_q, h_kv, num_blocks, slots, 3, _lib.ptr(seg), _lib.ptr(split),
              _lib.ptr(counts), seg_cap, max(seg_len, 1), MAX_SEGMENTS, _lib.ptr(ws),
              ws.numel(), _lib.stream_handle(dev))
    return CSCIndex(col_nnz=col_nnz, col_offsets=col_offsets, row_indices=row_indices,
                    head_indices=head_indices, slot_of_pair=slot_of_pair, order=order,
                    num_blocks=num_blocks, max_slots=slots, num_query_heads=h_q,
                    cu_seqlens=cu_seqlens, max_seqlen=max_seqlen, segments=seg,
                    seg_split=split, seg_counts=counts, seg_cap=seg_cap)


def build_csc_fused(q: torch.Tensor, k: torch.Tensor, cfg: MoBAConfig,
                    cu_seqlens: torch.Tensor | None = None,
                    max_seqlen: int | None = None) -> CSCIndex:
    """Pool -> gate -> transpose, all on the GPU, no host sync
    (`routing.py:430-464`)."""
    kbar = pool_blocks(k, cfg, cu_seqlens=cu_seqlens, max_seqlen=max_seqlen)
    block_idx = gate_select(q, kbar, cfg, cu_seqlens=cu_seqlens, max_seqlen=max_seqlen)
    return build_csc_from_indices(block_idx, kbar.shape[2], cfg, num_kv_heads=k.shape[2],
                                  cu_seqlens=cu_seqlens, max_seqlen=max_seqlen)


def csc_to_mask(index: CSCIndex, seq_len: int) -> torch.Tensor:
    """Expands an index back to a dense [B, H_q, S, nb] selection mask
    (`routing.py:564-624`); test support, synchronises with the host.

    Raises:
        ValueError: If col_offsets is not the exclusive prefix sum of col_nnz.
    """
    b, h_kv, n = index.col_nnz.shape
    packed = index.cu_seqlens is not None
    dev = index.col_nnz.device
    out = torch.zeros(1 if packed else b, index.num_query_heads, seq_len, n,
                      dtype=torch.bool, device=dev)
    prefix = index.col_nnz.cumsum(-1) - index.col_nnz
    if not torch.equal(prefix.to(index.col_offsets.dtype), index.col_offsets[..., :n]):
        raise ValueError("col_offsets is not the exclusive prefix sum of col_nnz; "
                         "the index is inconsistent")
    cols = torch.arange(n, device=dev)
    for bi in range(b):
        for kv in range(h_kv):
            blocks = torch.repeat_interleave(cols, index.col_nnz[bi, kv].long())
            total = blocks.numel()
            rows = index.row_indices[bi, kv, :total].long()
            heads = index.head_indices[bi, kv, :total].long()
            out[0 if packed else bi, heads, rows, blocks] = True
    return out
