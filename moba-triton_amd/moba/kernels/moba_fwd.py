"""KV-block-major forward (reference `src/moba/kernels/moba_fwd.py`).

`attend_partials` runs one program per (KV block, kv head): the block's keys
against every query that selected it, writing per-slot un-normalised
partials (m in log2 units, l, acc). `combine_partials` merges each query's
slots. Both run the HIP library.
"""

import torch

from moba import _lib
from moba.config import MoBAConfig
from moba.device import TENSOR_CORE_TILE, check_gathered_head_dim
from moba.gqa import head_group_size
from moba.kernels.routing import CSCIndex, build_csc_fused, index_stride
from moba.varlen import validate_cu_seqlens


def empty_partials(shape, slots: int, device, partials_dtype=torch.float32):
    """Uninitialised head-major partial buffers for a token-major query
    shape (`moba_fwd.py:529-563`): part_m, part_l [B, H, S, K] fp32 and
    part_acc [B, H, S, K, D] in `partials_dtype`.

    part_m and part_l are the two halves of one interleaved [B, H, S, K, 2]
    buffer, so that a slot's (m, l) pair is one 8-byte record in HBM.
    """
    b, s, h, d = shape
    ml = torch.empty((b, h, s, slots, 2), device=device, dtype=torch.float32)
    return (ml[..., 0], ml[..., 1],
            torch.empty((b, h, s, slots, d), device=device, dtype=partials_dtype))


def _interleaved(part_m, part_l) -> bool:
    """True when part_m / part_l are the halves of one (m, l) pair buffer
    as `empty_partials` makes them."""
    if part_m.dtype != torch.float32 or part_l.dtype != torch.float32:
        return False
    if part_m.shape != part_l.shape or part_m.stride() != part_l.stride():
        return False
    if part_l.data_ptr() != part_m.data_ptr() + 4:
        return False
    want, run = [], 2
    for n in reversed(part_m.shape):
        want.append(run)
        run *= n
    return all(st == w or n == 1 for st, w, n in
               zip(part_m.stride(), reversed(want), part_m.shape))


def pack_ml(part_m, part_l) -> torch.Tensor:
    """The (m, l) pair buffer [..., 2] fp32 for the library: the shared base
    of interleaved halves, else a packed copy."""
    if _interleaved(part_m, part_l):
        return torch.as_strided(part_m, tuple(part_m.shape) + (2,),
                                tuple(part_m.stride()) + (1,))
    return torch.stack((part_m.float(), part_l.float()), dim=-1).contiguous()


def _rows(index: CSCIndex, b: int) -> int:
    return index.col_nnz.shape[0]


def attend_partials(q, k, v, cfg: MoBAConfig, index: CSCIndex, causal: bool = True,
                    partials_dtype=None, partials=None):
    """The attention stage, returning un-merged partials (`moba_fwd.py:566-665`).

    part_m is reset to -inf inside the library call (the written-marker);
    part_l / part_acc of unwritten slots are never read. Caller-given
    `partials` must come from `empty_partials` (interleaved m / l halves).
    """
    b, s, h_q, d = q.shape
    h_kv = k.shape[2]
    dev = _lib.require_gpu(q, k, v)
    slots = index.max_slots
    if partials_dtype is None:
        partials_dtype = q.dtype
    if partials is None:
        partials = empty_partials(q.shape, slots, dev, partials_dtype)
    part_m, part_l, part_acc = partials
    if not _interleaved(part_m, part_l):
        raise ValueError("partials must come from empty_partials (interleaved m / l)")
    q, k, v = (_lib.aligned_contiguous(t) for t in (q, k, v))
    rows = _rows(index, b)
    mx = index.max_seqlen if index.cu_seqlens is not None else s
    _lib.call("moba_attend", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v),
              _lib.ptr(index.col_nnz), _lib.ptr(index.col_offsets),
              _lib.ptr(index.row_indices), _lib.ptr(index.head_indices),
              _lib.ptr(index.slot_of_pair), _lib.ptr(index.order),
              _lib.ptr(part_m), _lib.ptr(part_acc), _lib.ptr(index.cu_seqlens), rows, s, mx, h_q, h_kv, d,
              index.num_blocks, cfg.block_size, slots, index.row_indices.shape[-1],
              index_stride(index), _lib.ptr(index.segments), _lib.ptr(index.seg_split),
              _lib.ptr(index.seg_counts), index.seg_cap,
              int(bool(causal)), _lib.DTYPE_CODE[q.dtype],
              _lib.DTYPE_CODE[part_acc.dtype], _lib.stream_handle(dev))
    return part_m, part_l, part_acc


def combine_partials(part_m, part_l, part_acc, out_dtype, block_m=None,
                     return_lse: bool = False):
    """Merges per-slot partials into the output (`moba_fwd.py:668-725`).

    Returns:
        out [B, S, H, D] (`out_dtype`), plus lse [B, H, S] fp32 in log2
        units when `return_lse`.

    Raises:
        ValueError: If the buffers disagree on shape.
    """
    del block_m  # the HIP merge has a fixed tile
    b, h, s, slots = part_m.shape
    d = part_acc.shape[-1]
    if part_l.shape != part_m.shape:
        raise ValueError(f"shape mismatch: part_l {tuple(part_l.shape)} against "
                         f"part_m {tuple(part_m.shape)}")
    if part_acc.shape != (b, h, s, slots, d):
        raise ValueError(f"shape mismatch: part_acc {tuple(part_acc.shape)} against "
                         f"{(b, h, s, slots, d)}")
    dev = _lib.require_gpu(part_m, part_l, part_acc)
    ml = pack_ml(part_m, part_l)
    part_acc = part_acc.contiguous()
    out = torch.empty((b, s, h, d), device=dev, dtype=out_dtype)
    lse = torch.empty((b, h, s), device=dev, dtype=torch.float32) if return_lse else None
    _lib.call("moba_combine", _lib.ptr(ml), _lib.ptr(part_acc),
              _lib.ptr(out), _lib.ptr(lse), b, s, h, d, slots,
              _lib.DTYPE_CODE[part_acc.dtype], _lib.DTYPE_CODE[out_dtype],
              _lib.stream_handle(dev))
    return (out, lse) if return_lse else out


def _validate(q, k, v, cfg: MoBAConfig, cu_seqlens=None, max_seqlen=None) -> None:
    """Shape and configuration checks before any launch (`moba_fwd.py:733-780`).

    Raises:
        ValueError: On mismatched shapes, indivisible heads, bad packing
            metadata, an unsupported head_dim or dtype, or block_size < 16.
    """
    if k.shape != v.shape:
        raise ValueError(f"key/value shape mismatch: {k.shape}, {v.shape}")
    if q.shape[0] != k.shape[0] or q.shape[1] != k.shape[1] or q.shape[3] != k.shape[3]:
        raise ValueError(f"shape mismatch: {q.shape}, {k.shape}, {v.shape}")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError(f"dtype mismatch: {q.dtype}, {k.dtype}, {v.dtype}")
    head_group_size(q.shape[2], k.shape[2])
    if cu_seqlens is not None:
        if q.shape[0] != 1:
            raise ValueError(f"packed input must have batch 1, got {q.shape[0]}")
        if max_seqlen is None:
            raise ValueError("max_seqlen is required when cu_seqlens is given")
        validate_cu_seqlens(cu_seqlens, total_tokens=q.shape[1], max_seqlen=max_seqlen)
    if q.dtype not in _lib.DTYPE_CODE:
        raise ValueError(f"unsupported dtype {q.dtype}")
    ok, reason = check_gathered_head_dim(q.shape[-1], q.element_size())
    if not ok:
        raise ValueError(reason)
    if q.shape[-1] > MAX_HEAD_DIM:
        # The reference admits any power of two (moba_fwd.py:774-776); the
        # kernels here cover up to 1024 (MFMA at 64 and 128, FMA beyond).
        raise ValueError(f"head_dim {q.shape[-1]} above {MAX_HEAD_DIM} is not supported")
    if cfg.block_size < TENSOR_CORE_TILE:
        raise ValueError(f"block_size {cfg.block_size} below the MFMA tile minimum "
                         f"of {TENSOR_CORE_TILE}")
    ok, reason = fits_attend_lds(q.shape[-1], cfg.block_size, q.dtype)
    if not ok:
        raise ValueError(reason)


# Shapes the MFMA attend kernel covers; the others run the FMA attend kernel,
# which keeps a block's keys and values in LDS at the input's width, whole
# or (when they do not fit) one tile of keys at a time.
_MFMA_HEAD_DIMS, _MFMA_BLOCKS = (64, 128), (32, 64, 128)
_LDS_BYTES = 160 * 1024
MAX_HEAD_DIM = 1024


def fits_attend_lds(head_dim: int, block_size: int, dtype) -> tuple[bool, str]:
    """Whether the FMA attend kernel can run the shape (csrc/attn_simple.hip
    moba_attend): a group's 16 float32 query rows and score rows, plus at
    least one key row, within 160 KiB of LDS. Always true where the MFMA
    kernel takes the shape."""
    if (dtype in (torch.bfloat16, torch.float16) and head_dim in _MFMA_HEAD_DIMS
            and block_size in _MFMA_BLOCKS):
        return True, ""
    esize = torch.empty((), dtype=dtype).element_size()
    e = 16  # queries per group of the FMA kernel
    lds = 4 * (e * head_dim + e * block_size + 2 * e) + 4 * 3 * e + esize * head_dim
    if lds > _LDS_BYTES:
        return False, (f"block_size {block_size} x head_dim {head_dim} in {dtype}: a group's "
                       f"queries and scores need {lds} bytes of LDS, above the {_LDS_BYTES} "
                       f"the attend kernel has")
    return True, ""


def moba_forward(q, k, v, cfg: MoBAConfig, index: CSCIndex | None = None,
                 causal: bool = True, partials_dtype=None, cu_seqlens=None,
                 max_seqlen=None):
    """MoBA attention forward, no autograd (`moba_fwd.py:783-835`)."""
    if index is not None:
        cu_seqlens, max_seqlen = index.cu_seqlens, index.max_seqlen
    _validate(q, k, v, cfg, cu_seqlens, max_seqlen)
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    if index is not None:
        part_m, part_l, part_acc = attend_partials(q, k, v, cfg, index, causal=causal,
                                                   partials_dtype=partials_dtype)
        return combine_partials(part_m, part_l, part_acc, q.dtype)
    # Without a caller's index the per-slot buffers are bounded by running
    # (batch row, kv head[, query heads]) chunks (moba.chunking).
    from moba.chunking import query_heads
    from moba.kernels.attention import _piece, forward_chunks
    chunks = forward_chunks(q, k, v, cfg, causal, cu_seqlens, max_seqlen,
                            partials_dtype=partials_dtype)
    group = q.shape[2] // k.shape[2]
    out = torch.empty_like(q) if len(chunks) > 1 else None
    for chunk in chunks:
        b0, b1, hk0, hk1 = chunk[:4]
        hq0, hq1 = query_heads(chunk, group)
        whole = len(chunks) == 1
        qc = q if whole else _piece(q, b0, b1, hq0, hq1)
        kc = k if whole else _piece(k, b0, b1, hk0, hk1)
        vc = v if whole else _piece(v, b0, b1, hk0, hk1)
        idx = build_csc_fused(qc, kc, cfg, cu_seqlens=cu_seqlens, max_seqlen=max_seqlen)
        part_m, part_l, part_acc = attend_partials(qc, kc, vc, cfg, idx, causal=causal,
                                                   partials_dtype=partials_dtype)
        oc = combine_partials(part_m, part_l, part_acc, q.dtype)
        if whole:
            return oc
        out[b0:b1, :, hq0:hq1] = oc
    return out
