"""MoBA attention as one differentiable operation
(reference `src/moba/kernels/attention.py`).

Saved for backward: q, k, v, out, lse (log2 units) and part_m (the
written-marker of the per-slot partials); the CSC index rides on ctx. The
gate receives no gradient (`attention.py:33-38`): routing is a hard top-k.
"""

import torch

from moba.config import MoBAConfig
from moba.kernels.moba_bwd import moba_backward
from moba.kernels.moba_fwd import _validate, attend_partials, combine_partials
from moba.kernels.routing import CSCIndex, build_csc_fused


class MoBAAttentionFunction(torch.autograd.Function):
    """Differentiable MoBA attention over the HIP kernels (`attention.py:53-92`)."""

    @staticmethod
    def forward(ctx, q, k, v, cfg, index, causal, cu_seqlens, max_seqlen):
        if index is not None:
            cu_seqlens, max_seqlen = index.cu_seqlens, index.max_seqlen
        _validate(q, k, v, cfg, cu_seqlens, max_seqlen)
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        if index is None:
            index = build_csc_fused(q, k, cfg, cu_seqlens=cu_seqlens, max_seqlen=max_seqlen)
        part_m, part_l, part_acc = attend_partials(q, k, v, cfg, index, causal=causal)
        out, lse = combine_partials(part_m, part_l, part_acc, q.dtype, return_lse=True)
        ctx.save_for_backward(q, k, v, out, lse, part_m)
        ctx.cfg, ctx.index, ctx.causal = cfg, index, causal
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse, part_m = ctx.saved_tensors
        dq, dk, dv = moba_backward(dout, q, k, v, out, lse, part_m, ctx.cfg, ctx.index,
                                   causal=ctx.causal)
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
