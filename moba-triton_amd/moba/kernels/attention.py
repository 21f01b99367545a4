"""MoBA attention as one differentiable operation
(reference `src/moba/kernels/attention.py`).

Saved for backward: q, k, v, out and, per chunk, lse (log2 units), part_m
(the written-marker of the per-slot partials) and the CSC index. The gate
receives no gradient (`attention.py:33-38`): routing is a hard top-k.
"""

import torch

from moba import _lib
from moba.chunking import partials_budget, plan_call, query_heads
from moba.config import MoBAConfig
from moba.kernels.moba_bwd import moba_backward
from moba.kernels.moba_fwd import _validate, attend_partials, combine_partials
from moba.kernels.routing import CSCIndex, build_csc_fused


def _piece(t, b0, b1, h0, h1):
    """t[b0:b1, :, h0:h1] as a contiguous tensor (a view when it already is)."""
    return t[b0:b1, :, h0:h1].contiguous()


def forward_chunks(q, k, v, cfg, causal, cu_seqlens, max_seqlen, partials_dtype=None):
    """The chunks (b0, b1, hk0, hk1, j0, j1) -- batch rows, kv heads, and
    query heads within each kv head's group -- the per-slot buffers of this
    call are split into (one chunk when they fit the budget of
    `moba.chunking`).

    The per-slot buffers are [B, Hq, S, slots(, D)] over the tensor's token
    axis, so a unit (one batch row, one kv head) spans all S tokens of the
    row; packed input is one row of T = S tokens, whatever max_seqlen is.
    Value rows are sized in the larger of q's dtype (the dQ partials) and
    `partials_dtype` (the forward's part_acc)."""
    _lib.require_gpu(q, k, v)  # raises before any device query on host tensors
    h_kv = k.shape[2]
    elem = q.element_size()
    if partials_dtype is not None:
        elem = max(elem, torch.empty((), dtype=partials_dtype).element_size())
    return plan_call(tuple(q.shape), h_kv, cfg.slots(), elem, partials_budget(q.device))


class MoBAAttentionFunction(torch.autograd.Function):
    """Differentiable MoBA attention over the HIP kernels (`attention.py:53-92`).

    Without a caller's index, a call whose per-slot buffers exceed the
    budget of `moba.chunking` runs chunk by chunk over (batch row, kv head)
    units, forward and backward, with the same results; a unit too large on
    its own is split by query head (dK / dV then summed in float32).
    """

    @staticmethod
    def forward(ctx, q, k, v, cfg, index, causal, cu_seqlens, max_seqlen):
        if index is not None:
            cu_seqlens, max_seqlen = index.cu_seqlens, index.max_seqlen
        _validate(q, k, v, cfg, cu_seqlens, max_seqlen)
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        group = q.shape[2] // k.shape[2]
        chunks = [(0, q.shape[0], 0, k.shape[2], 0, group)] if index is not None else \
            forward_chunks(q, k, v, cfg, causal, cu_seqlens, max_seqlen)
        out = torch.empty_like(q) if len(chunks) > 1 else None
        saved = []
        for chunk in chunks:
            b0, b1, hk0, hk1 = chunk[:4]
            hq0, hq1 = query_heads(chunk, group)
            whole = len(chunks) == 1
            qc = q if whole else _piece(q, b0, b1, hq0, hq1)
            kc = k if whole else _piece(k, b0, b1, hk0, hk1)
            vc = v if whole else _piece(v, b0, b1, hk0, hk1)
            idx = index if index is not None else build_csc_fused(
                qc, kc, cfg, cu_seqlens=cu_seqlens, max_seqlen=max_seqlen)
            part_m, part_l, part_acc = attend_partials(qc, kc, vc, cfg, idx, causal=causal)
            oc, lse = combine_partials(part_m, part_l, part_acc, q.dtype, return_lse=True)
            del part_l, part_acc
            if whole:
                out = oc
            else:
                out[b0:b1, :, hq0:hq1] = oc
            saved.append((idx, lse, part_m))
        ctx.save_for_backward(q, k, v, out)
        ctx.cfg, ctx.causal, ctx.chunks, ctx.saved = cfg, causal, chunks, saved
        ctx.index = saved[0][0] if len(chunks) == 1 else None
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out = ctx.saved_tensors
        chunks, group = ctx.chunks, q.shape[2] // k.shape[2]
        if len(chunks) == 1:
            idx, lse, part_m = ctx.saved[0]
            dq, dk, dv = moba_backward(dout, q, k, v, out, lse, part_m, ctx.cfg, idx,
                                       causal=ctx.causal)
            return dq, dk, dv, None, None, None, None, None
        # Chunks holding part of a kv head's group add their unrounded
        # float32 dK / dV; the sum is rounded once.
        split = any((c[4], c[5]) != (0, group) for c in chunks)
        dq = torch.empty_like(q)
        dk, dv = ((torch.zeros(k.shape, dtype=torch.float32, device=k.device),
                   torch.zeros(v.shape, dtype=torch.float32, device=v.device)) if split
                  else (torch.empty_like(k), torch.empty_like(v)))
        for chunk, (idx, lse, part_m) in zip(chunks, ctx.saved):
            b0, b1, hk0, hk1 = chunk[:4]
            hq0, hq1 = query_heads(chunk, group)
            g = moba_backward(_piece(dout, b0, b1, hq0, hq1), _piece(q, b0, b1, hq0, hq1),
                              _piece(k, b0, b1, hk0, hk1), _piece(v, b0, b1, hk0, hk1),
                              _piece(out, b0, b1, hq0, hq1), lse, part_m, ctx.cfg, idx,
                              causal=ctx.causal, dkv_dtype=torch.float32 if split else None)
            dq[b0:b1, :, hq0:hq1] = g[0]
            if split:
                dk[b0:b1, :, hk0:hk1] += g[1]
                dv[b0:b1, :, hk0:hk1] += g[2]
            else:
                dk[b0:b1, :, hk0:hk1] = g[1]
                dv[b0:b1, :, hk0:hk1] = g[2]
        if split:
            dk, dv = dk.to(k.dtype), dv.to(v.dtype)
        return dq, dk, dv, None, None, None, None, None


def moba_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cfg: MoBAConfig,
                   index: CSCIndex | None = None, causal: bool = True,
                   cu_seqlens: torch.Tensor | None = None,
                   max_seqlen: int | None = None) -> torch.Tensor:
    """MoBA attention with gradient support (`attention.py:95-132`).

    Args:
        q: [B, S, H_q, D]; k, v: [B, S, H_kv, D] with H_kv dividing H_q.
        cfg: Configuration.
        index: Precomputed CSC index (holds routing fixed); built on the GPU
            when omitted.
        causal: Causal mask inside the query's own block.
        cu_seqlens / max_seqlen: Packed mode ([1, T, H, D] inputs).
    """
    return MoBAAttentionFunction.apply(q, k, v, cfg, index, causal, cu_seqlens, max_seqlen)
