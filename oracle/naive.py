"""Torch restatement of the reference MoBA oracle (test infrastructure only).

Every function names the reference lines it restates. Inputs are token-major
`[B, S, H, D]`; internal buffers (block representatives, masks, partials,
index columns) are head-major, as in the reference (`src/moba/gqa.py:55-62`).

The config argument is duck-typed: anything with `block_size`, `top_k`,
`always_select_current`, `top_k_includes_current`, `tie_break_low_index`.
"""

from __future__ import annotations

import math

import torch

__all__ = [
    "num_blocks", "past_blocks_selected", "head_group_size", "expand_kv",
    "round_to_dtype", "pool_blocks", "gate_scores", "select_from_scores",
    "gate_select", "moba_selection", "mask_to_indices", "indices_to_mask",
    "moba_attention", "moba_attention_sparse", "build_csc", "csc_to_mask",
    "combine_reference", "slots_per_query", "sparse_grads",
    "super_block_means", "hierarchical_select",
]


# ---------------------------------------------------------------------------
# Config arithmetic  (src/moba/config.py:69-99)
# ---------------------------------------------------------------------------


def num_blocks(seq_len: int, block_size: int) -> int:
    """ceil(seq_len / block_size), `config.py:86-99`."""
    return -(-seq_len // block_size)


def past_blocks_selected(cfg, n_blocks: int) -> int:
    """Past-block budget, `config.py:69-84`: top_k, minus one when the own
    block is forced and counts against top_k; clamped to [0, n_blocks]."""
    budget = cfg.top_k
    if cfg.always_select_current and cfg.top_k_includes_current:
        budget -= 1
    return max(0, min(budget, n_blocks))


def slots_per_query(cfg) -> int:
    """Most blocks one query can select: the past budget plus the own block.

    Equals `top_k` under the default flags, which is the reference's
    `CSCIndex.max_slots` (`routing.py:422`).
    """
    budget = cfg.top_k
    if cfg.always_select_current and cfg.top_k_includes_current:
        budget -= 1
    return budget + (1 if cfg.always_select_current else 0)


# ---------------------------------------------------------------------------
# GQA  (src/moba/gqa.py:22-84)
# ---------------------------------------------------------------------------


def head_group_size(h_q: int, h_kv: int) -> int:
    """`gqa.py:22-46`: positive counts, h_q a multiple of h_kv."""
    if h_q <= 0 or h_kv <= 0:
        raise ValueError(f"head counts must be positive, got q={h_q} kv={h_kv}")
    if h_q % h_kv:
        raise ValueError(f"query heads {h_q} not divisible by kv heads {h_kv}")
    return h_q // h_kv


def expand_kv(t: torch.Tensor, h_q: int, dim: int = 2) -> torch.Tensor:
    """`gqa.py:49-84`: query head g reads kv head g // group."""
    group = head_group_size(h_q, t.shape[dim])
    return t if group == 1 else t.repeat_interleave(group, dim=dim)


# ---------------------------------------------------------------------------
# Rounding
# ---------------------------------------------------------------------------


def round_to_dtype(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Rounds an (exact, float64) value the way a float32-accumulating BLAS
    that returns `dtype` would: once to float32, then to `dtype`.

    float64 inputs stay float64 (the reference runs its Tier-1 identities in
    float64, `tests/test_semantics.py:1-8`).
    """
    if dtype == torch.float64:
        return x.to(torch.float64)
    return x.to(torch.float32).to(dtype)


# ---------------------------------------------------------------------------
# Pooling  (src/moba/naive.py:23-61, kernels/pooling.py:82-93)
# ---------------------------------------------------------------------------


def pool_blocks(k: torch.Tensor, block_size: int) -> torch.Tensor:
    """Block-mean keys, `[B, S, H, D] -> [B, H, n_blocks, D]`.

    Restates `naive.py:49-61`: pad to a block multiple, sum each block, divide
    by the block's real occupancy (a short tail divides by its own count).
    Rounding follows `pooling.py:82-93`: the sum is rounded to the input dtype
    before the divide, and the quotient is rounded again. The sum is taken in
    float64 (exact for 128 bf16 terms), see the package docstring.
    """
    b, s, h, d = k.shape
    n = num_blocks(s, block_size)
    pad = n * block_size - s
    kd = torch.nn.functional.pad(k.to(torch.float64), (0, 0, 0, 0, 0, pad))
    sums = kd.view(b, n, block_size, h, d).sum(dim=2).transpose(1, 2)
    counts = torch.full((n,), float(block_size), dtype=torch.float64)
    counts[-1] = block_size - pad
    counts = counts.view(1, 1, n, 1)
    if k.dtype == torch.float64:
        return sums / counts
    sums_r = round_to_dtype(sums, k.dtype).to(torch.float32)
    return (sums_r / counts.to(torch.float32)).to(k.dtype)


# ---------------------------------------------------------------------------
# Gate  (src/moba/naive.py:64-146)
# ---------------------------------------------------------------------------


def gate_scores(q: torch.Tensor, kbar: torch.Tensor,
                chunk: int = 4096) -> torch.Tensor:
    """Unscaled gate scores `[B, H_q, S, n]`, correctly rounded to q.dtype.

    Restates `naive.py:103-109` (`einsum('bshd,bhnd->bhsn')`, kbar expanded
    over the group, no 1/sqrt(D) since a monotone scale cannot reorder a
    ranking). The dot product is exact in float64 and then rounded once to
    float32 and once to the input dtype.
    """
    b, s, h, _ = q.shape
    kb = expand_kv(kbar, h, dim=1).to(torch.float64)
    out = torch.empty(b, h, s, kbar.shape[2], dtype=q.dtype)
    for lo in range(0, s, chunk):
        hi = min(lo + chunk, s)
        exact = torch.einsum("bshd,bhnd->bhsn", q[:, lo:hi].to(torch.float64), kb)
        out[:, :, lo:hi] = round_to_dtype(exact, q.dtype)
    return out


def select_from_scores(scores: torch.Tensor, cfg, pos=None) -> torch.Tensor:
    """Selection mask `[B, H, S, n]` from gate scores, `naive.py:111-146`.

    Candidates are blocks strictly before the query's own block; a stable
    descending sort ranks them so equal scores favour the lower block index;
    the first `past_blocks_selected(n)` survive, -inf leftovers are dropped,
    and the own block is OR-ed in when forced. `pos` gives the sequence
    position of each score row (default: row r is position r).
    """
    b, h, s, n = scores.shape
    pos = torch.arange(s) if pos is None else torch.as_tensor(pos, dtype=torch.int64)
    own = pos // cfg.block_size
    blocks = torch.arange(n)
    is_past = blocks.view(1, -1) < own.view(-1, 1)
    is_cur = blocks.view(1, -1) == own.view(-1, 1)
    masked = scores.masked_fill(~is_past.view(1, 1, s, n), float("-inf"))
    order = torch.argsort(masked, dim=-1, descending=True,
                          stable=bool(cfg.tie_break_low_index))
    take = past_blocks_selected(cfg, n)
    sel = torch.zeros_like(masked, dtype=torch.bool)
    sel.scatter_(-1, order[..., :take], True)
    sel &= is_past.view(1, 1, s, n)
    if cfg.always_select_current:
        sel |= is_cur.view(1, 1, s, n)
    return sel


def gate_select(q: torch.Tensor, kbar: torch.Tensor, cfg) -> torch.Tensor:
    """`naive.py:64-146` with this oracle's score rounding."""
    return select_from_scores(gate_scores(q, kbar), cfg)


def gate_select_rows(q: torch.Tensor, kbar: torch.Tensor, cfg, rows) -> torch.Tensor:
    """`gate_select(q, kbar, cfg)[:, :, rows]` without scoring the other rows:
    the selection of a query depends only on its own row and position, so the
    same scores and ranking restricted to `rows` (positions in one sequence)
    give the same mask `[B, H, len(rows), n]`. For full-length sequences where
    the dense `[S, n]` score matrix would not fit."""
    rows = torch.as_tensor(rows, dtype=torch.int64)
    return select_from_scores(gate_scores(q[:, rows], kbar), cfg, pos=rows)


def super_block_means(kbar: torch.Tensor, group: int) -> torch.Tensor:
    """Super-block representatives `[B, H, ceil(n / group), D]`: the blocks'
    representatives pooled `group` at a time exactly as `pool_blocks` pools
    keys (sum rounded to the dtype, divided by the real count, a short tail
    by its own). This build's definition for the opt-in hierarchical gate;
    the reference's probe pooled the same way in spirit
    (`docs/gate-hierarchical-measurements.md`, "mean-pooled super-block
    representatives")."""
    return pool_blocks(kbar.transpose(1, 2), group)


def hierarchical_select(q: torch.Tensor, kbar: torch.Tensor, cfg, group: int,
                        opened: int, rows=None) -> torch.Tensor:
    """Coarse-to-fine selection mask `[B, H, S, n]` (opt-in; never the
    default). Restates the scheme of `docs/gate-hierarchical-measurements.md`
    (group blocks into super-blocks of `group`, score the super-block
    representatives, open the best `opened`, score only the blocks inside):

    1. the super-block gate: `gate_select` over `super_block_means(kbar,
       group)` with block size `block_size * group`, `opened` strictly-past
       super-blocks plus the query's own super-block;
    2. candidates: the strictly-past blocks inside those super-blocks;
    3. the usual ranking (`select_from_scores`: exact score rounded to
       float32 and to the dtype, ties to the lower block) over the
       candidates only; the own block forced as usual.
    With `opened` >= the number of super-blocks, or `group` 1 and `opened` >=
    the past budget, this is `gate_select` exactly. `rows` restricts the
    result to those query positions (`[B, H, len(rows), n]`), as
    `gate_select_rows` does.
    """
    from types import SimpleNamespace
    n = kbar.shape[2]
    pos = torch.arange(q.shape[1]) if rows is None else torch.as_tensor(rows, dtype=torch.int64)
    qr = q if rows is None else q[:, pos]
    scfg = SimpleNamespace(block_size=cfg.block_size * group, top_k=opened + 1,
                           always_select_current=True, top_k_includes_current=True,
                           tie_break_low_index=True)
    sup = select_from_scores(gate_scores(qr, super_block_means(kbar, group)), scfg, pos=pos)
    cand = sup[..., torch.arange(n) // group]                         # [B, H, R, n]
    scores = gate_scores(qr, kbar).masked_fill(~cand, float("-inf"))
    sel = select_from_scores(scores, cfg, pos=pos)
    own = (pos // cfg.block_size).view(1, 1, -1, 1)
    return sel & (cand | (torch.arange(n).view(1, 1, 1, n) == own))


def moba_selection(q, k, cfg, cu_seqlens=None) -> torch.Tensor:
    """Pool then gate, `naive.py:149-189`.

    Packed (`cu_seqlens` given, batch 1): each sequence is gated alone, block
    ids are sequence-local, and the block axis is as wide as the longest
    sequence's block count (`naive.py:175-189`).
    """
    if cu_seqlens is None:
        return gate_select(q, pool_blocks(k, cfg.block_size), cfg)
    if q.shape[0] != 1:
        raise ValueError(f"packed input must have batch 1, got {q.shape[0]}")
    bounds = [int(x) for x in cu_seqlens.tolist()]
    spans = list(zip(bounds[:-1], bounds[1:]))
    width = max(num_blocks(hi - lo, cfg.block_size) for lo, hi in spans)
    out = torch.zeros(1, q.shape[2], q.shape[1], width, dtype=torch.bool)
    for lo, hi in spans:
        piece = moba_selection(q[:, lo:hi], k[:, lo:hi], cfg)
        out[:, :, lo:hi, :piece.shape[-1]] = piece
    return out


def mask_to_indices(mask: torch.Tensor, slots: int) -> torch.Tensor:
    """Dense mask -> ids `[B, H, S, slots]` int32, ascending, -1 padded.

    The gate's output contract (`gating.py:300-335`, `tests/test_gate.py:69-92`):
    slot j holds the query's j-th selection by ascending block id.
    """
    n = mask.shape[-1]
    ids = torch.arange(n, dtype=torch.int64).expand_as(mask)
    key = torch.where(mask, ids, torch.full_like(ids, n))
    srt = key.sort(dim=-1).values[..., :slots]
    if srt.shape[-1] < slots:
        pad = torch.full(srt.shape[:-1] + (slots - srt.shape[-1],), n)
        srt = torch.cat([srt, pad], dim=-1)
    return torch.where(srt < n, srt, torch.full_like(srt, -1)).to(torch.int32)


def indices_to_mask(idx: torch.Tensor, n: int) -> torch.Tensor:
    """Ids -> mask, padding routed to a dropped scratch column
    (`tests/test_gate.py:25-47`)."""
    b, h, s, _ = idx.shape
    m = torch.zeros(b, h, s, n + 1, dtype=torch.bool)
    tgt = torch.where(idx >= 0, idx.long(), torch.full_like(idx.long(), n))
    m.scatter_(-1, tgt, True)
    return m[..., :n]


# ---------------------------------------------------------------------------
# Attention  (src/moba/naive.py:234-329)
# ---------------------------------------------------------------------------


def moba_attention(q, k, v, cfg, selected=None, query_chunk=None,
                   cu_seqlens=None) -> torch.Tensor:
    """Dense masked-softmax MoBA attention, `naive.py:234-329`.

    Token visibility is the block selection broadcast over each block's keys,
    intersected with the causal mask; logits are scaled by D^-1/2. Computed in
    q's dtype (pass float64 tensors for ground truth). Packed input attends
    per sequence (`naive.py:210-231`). Differentiable.
    """
    if cu_seqlens is not None:
        if q.shape[0] != 1:
            raise ValueError(f"packed input must have batch 1, got {q.shape[0]}")
        bounds = [int(x) for x in cu_seqlens.tolist()]
        pieces = []
        for lo, hi in zip(bounds[:-1], bounds[1:]):
            sel = None
            if selected is not None:
                sel = selected[:, :, lo:hi, :num_blocks(hi - lo, cfg.block_size)]
            pieces.append(moba_attention(q[:, lo:hi], k[:, lo:hi], v[:, lo:hi],
                                         cfg, selected=sel,
                                         query_chunk=query_chunk))
        return torch.cat(pieces, dim=1)

    b, s, h, d = q.shape
    scale = d ** -0.5
    k, v = expand_kv(k, h), expand_kv(v, h)
    if selected is None:
        selected = moba_selection(q, k, cfg)
    pos = torch.arange(s)
    blk = pos // cfg.block_size
    step = s if query_chunk is None else min(query_chunk, s)
    outs = []
    for lo in range(0, s, step):
        hi = min(lo + step, s)
        vis = selected[:, :, lo:hi][..., blk]
        causal = pos[lo:hi].view(-1, 1) >= pos.view(1, -1)
        mask = vis & causal.view(1, 1, hi - lo, s)
        logits = torch.einsum("bihd,bjhd->bhij", q[:, lo:hi], k) * scale
        logits = logits.masked_fill(~mask, float("-inf"))
        probs = torch.softmax(logits, dim=-1)
        outs.append(torch.einsum("bhij,bjhd->bihd", probs, v))
    return torch.cat(outs, dim=1)


def moba_attention_sparse(q, k, v, block_idx, block_size, rows=None,
                          bos=0, causal=True):
    """Gather form of the same attention for long sequences.

    For each query (optionally only the positions in `rows`) gathers the keys
    of its selected blocks (`block_idx` `[B, H_q, S, slots]`, -1 padded,
    sequence-local ids relative to token `bos`), applies the causal mask and
    a softmax. Same definition as `moba_attention`; cost O(S * slots * bs * D).
    Returns `(out [B, R, H, D], lse [B, H, R])`, lse in natural-log units,
    computed in q's dtype (use float64). Differentiable.
    """
    b, s, h, d = q.shape
    h_kv = k.shape[2]
    g = head_group_size(h, h_kv)
    if rows is None:
        rows = torch.arange(s)
    rows = torch.as_tensor(rows, dtype=torch.int64)
    r = rows.numel()
    slots = block_idx.shape[-1]
    scale = d ** -0.5
    hq = torch.arange(h)
    idx = block_idx[:, :, rows].long()                      # [B,H,R,slots]
    valid_blk = idx >= 0
    key_off = torch.arange(block_size)
    kpos = bos + idx.clamp(min=0)[..., None] * block_size + key_off  # [B,H,R,sl,bs]
    kpos_local = kpos - bos
    in_seq = kpos < s
    qpos = rows.view(1, 1, r, 1, 1)
    ok = valid_blk[..., None] & in_seq
    if causal:
        ok = ok & (kpos_local <= (qpos - bos))
    kp = kpos.clamp(max=s - 1).reshape(b, h, r * slots * block_size)
    bi = torch.arange(b).view(b, 1, 1)
    kvh = (hq // g).view(1, h, 1)
    kk = k[bi, kp, kvh].view(b, h, r, slots * block_size, d)
    vv = v[bi, kp, kvh].view(b, h, r, slots * block_size, d)
    qq = q[:, rows].permute(0, 2, 1, 3)                     # [B,H,R,D]
    logits = torch.einsum("bhrd,bhrjd->bhrj", qq, kk) * scale
    logits = logits.masked_fill(~ok.view(b, h, r, -1), float("-inf"))
    lse = torch.logsumexp(logits, dim=-1)
    probs = torch.exp(logits - lse[..., None])
    out = torch.einsum("bhrj,bhrjd->bhrd", probs, vv)
    return out.permute(0, 2, 1, 3), lse


def sparse_grads(q, k, v, do, block_idx, block_size, rows, key_blocks=None,
                 dtype=torch.float64, max_gather_bytes=1 << 30, key_users_only=False):
    """Explicit gradients of (out * dO).sum() for the query rows `rows` of a
    batch-1 sequence, without autograd: the same attention as
    `moba_attention_sparse` differentiated by hand, in the backward's
    formulation (reference `src/moba/kernels/moba_bwd.py:216-394`):
    p = softmax(q.K * D^-1/2), O = p.V, delta = O.dO, dp = dO.V,
    ds = p (dp - delta), dq = ds.K * D^-1/2, dK += ds^T q * D^-1/2,
    dV += p^T dO.

    Every product is formed in `dtype` (float64 for ground truth; bfloat16
    gives the same-dtype oracle of the tolerance policy) and every sum over
    queries (dK, dV) or keys (dq, O) is accumulated in float32 or float64 and
    rounded once to `dtype`, as one matmul in that dtype would be.

    Only rows whose queries appear in `rows` contribute; dK / dV are
    accumulated for the keys of `key_blocks` (block ids; None = every key).
    Returns (out [1, R, H, D], dq [1, R, H, D], dk [1, S, Hkv, D],
    dv [1, S, Hkv, D]) in `dtype`; dk / dv hold zeros outside `key_blocks`.
    With `key_users_only`, a (row, head) pair whose selection holds none of
    `key_blocks` is skipped (it adds nothing to those keys) and its out / dq
    stay zero.
    """
    b, s, h, d = q.shape
    if b != 1:
        raise ValueError("sparse_grads takes one sequence (batch 1)")
    h_kv = k.shape[2]
    g = head_group_size(h, h_kv)
    acc_t = torch.float64 if dtype == torch.float64 else torch.float32
    scale = torch.tensor(d ** -0.5, dtype=dtype)
    rows = torch.as_tensor(rows, dtype=torch.int64)
    r_all = rows.numel()
    slots = block_idx.shape[-1]
    width = slots * block_size
    dk = torch.zeros(s, h_kv, d, dtype=acc_t)
    dv = torch.zeros(s, h_kv, d, dtype=acc_t)
    out = torch.zeros(r_all, h, d, dtype=dtype)
    dq = torch.zeros(r_all, h, d, dtype=dtype)
    qx, kx, vx, dox = (t[0].to(dtype) for t in (q, k, v, do))
    keys_wanted = None
    if key_blocks is not None:
        keys_wanted = torch.zeros(-(-s // block_size) + 1, dtype=torch.bool)
        keys_wanted[torch.as_tensor(key_blocks, dtype=torch.int64)] = True
    chunk = max(1, max_gather_bytes // (width * d * 8 * 2))
    key_off = torch.arange(block_size)
    for hq in range(h):
        hk = hq // g
        k_h, v_h = kx[:, hk].contiguous(), vx[:, hk].contiguous()
        todo = torch.arange(r_all)
        if key_users_only and keys_wanted is not None:
            ids = block_idx[0, hq, rows].long()
            todo = torch.nonzero(((ids >= 0) & keys_wanted[ids.clamp(min=0)]).any(-1)).flatten()
        for lo in range(0, todo.numel(), chunk):
            sel = todo[lo:lo + chunk]
            r = rows[sel]
            blk = block_idx[0, hq, r].long()                              # [R, slots]
            kpos = blk.clamp(min=0)[..., None] * block_size + key_off     # [R, slots, bs]
            ok = (blk >= 0)[..., None] & (kpos < s) & (kpos <= r.view(-1, 1, 1))
            kpos = kpos.clamp(max=s - 1).reshape(-1, width)
            ok = ok.reshape(-1, width)
            flat = kpos.reshape(-1)
            kg = k_h.index_select(0, flat).view(-1, width, d)             # [R, W, D]
            vg = v_h.index_select(0, flat).view(-1, width, d)
            qr, dor = qx[r, hq], dox[r, hq]                               # [R, D]
            logits = torch.einsum("rd,rwd->rw", qr, kg) * scale
            logits = logits.masked_fill(~ok, float("-inf"))
            p = torch.softmax(logits.to(acc_t), dim=-1).to(dtype)
            o = torch.einsum("rw,rwd->rd", p, vg)
            delta = (o.to(acc_t) * dor.to(acc_t)).sum(-1, keepdim=True).to(dtype)
            dp = torch.einsum("rd,rwd->rw", dor, vg)
            ds = p * (dp - delta)
            out[sel, hq] = o
            dq[sel, hq] = (torch.einsum("rw,rwd->rd", ds.to(acc_t), kg.to(acc_t))
                           * scale.to(acc_t)).to(dtype)
            live = ok
            if keys_wanted is not None:
                live = live & keys_wanted[blk.clamp(min=0)].repeat_interleave(block_size, -1)
            if not bool(live.any()):
                continue
            rr, ww = torch.nonzero(live, as_tuple=True)
            kp = kpos[rr, ww]
            dk_c = (ds[rr, ww, None] * qr[rr] * scale).to(dtype)
            dv_c = (p[rr, ww, None] * dor[rr]).to(dtype)
            dk[:, hk].index_add_(0, kp, dk_c.to(acc_t))
            dv[:, hk].index_add_(0, kp, dv_c.to(acc_t))
    return (out.unsqueeze(0), dq.unsqueeze(0), dk.to(dtype).unsqueeze(0),
            dv.to(dtype).unsqueeze(0))


# ---------------------------------------------------------------------------
# CSC transpose  (src/moba/kernels/routing.py:467-624)
# ---------------------------------------------------------------------------


def build_csc(mask: torch.Tensor, h_kv: int, slots: int) -> dict:
    """Reference CSC builder from a dense mask, `routing.py:467-561`.

    Columns are keyed by (batch, kv head, block); entries are ordered by
    (query head within the group, position); a pair's slot is the block's
    rank among the query's selections by ascending id; `order` is a stable
    descending argsort of the column counts (longest first, lower id on ties).
    """
    b, h_q, s, n = mask.shape
    g = head_group_size(h_q, h_kv)
    total = g * s * slots
    slot_grid = (mask.to(torch.int64).cumsum(-1) - 1)
    stacked = mask.view(b, h_kv, g, s, n)
    col_nnz = stacked.sum(dim=(2, 3)).to(torch.int32)
    col_offsets = torch.zeros(b, h_kv, n + 1, dtype=torch.int32)
    col_offsets[..., 1:] = col_nnz.cumsum(-1)
    rows = torch.zeros(b, h_kv, total, dtype=torch.int32)
    heads = torch.zeros(b, h_kv, total, dtype=torch.int32)
    slot_of = torch.zeros(b, h_kv, total, dtype=torch.int32)
    for bi in range(b):
        for kv in range(h_kv):
            m = stacked[bi, kv].permute(2, 0, 1)           # [n, g, s]
            nz = m.reshape(-1).nonzero().squeeze(1)
            col = nz // (g * s)
            rem = nz % (g * s)
            gg = rem // s
            ss = rem % s
            cnt = nz.numel()
            rows[bi, kv, :cnt] = ss.to(torch.int32)
            heads[bi, kv, :cnt] = (kv * g + gg).to(torch.int32)
            slot_of[bi, kv, :cnt] = slot_grid[bi, kv * g + gg, ss, col].to(torch.int32)
    order = torch.argsort(col_nnz.to(torch.int64), dim=-1, descending=True,
                          stable=True).to(torch.int32)
    return dict(col_nnz=col_nnz, col_offsets=col_offsets, row_indices=rows,
                head_indices=heads, slot_of_pair=slot_of, order=order)


def csc_to_mask(col_nnz, col_offsets, row_indices, head_indices,
                num_query_heads: int, seq_len: int, packed: bool = False):
    """Inverse of the transpose, `routing.py:564-624`: checks that offsets
    are the exclusive prefix sum of counts, then scatters each column's
    (head, row) entries back into a `[B, H_q, S, n]` mask."""
    b, h_kv, n = col_nnz.shape
    prefix = col_nnz.to(torch.int64).cumsum(-1) - col_nnz.to(torch.int64)
    if not torch.equal(prefix.to(col_offsets.dtype), col_offsets[..., :n]):
        raise ValueError("col_offsets is not the exclusive prefix sum of col_nnz")
    out = torch.zeros(1 if packed else b, num_query_heads, seq_len, n,
                      dtype=torch.bool)
    cols = torch.arange(n)
    for bi in range(b):
        for kv in range(h_kv):
            blocks = torch.repeat_interleave(cols, col_nnz[bi, kv].long())
            t = blocks.numel()
            r = row_indices[bi, kv, :t].long()
            hh = head_indices[bi, kv, :t].long()
            out[0 if packed else bi, hh, r, blocks] = True
    return out


# ---------------------------------------------------------------------------
# Merge  (tests/test_moba_kernel.py:117-139, kernels/moba_fwd.py:429-521)
# ---------------------------------------------------------------------------


def combine_reference(part_m, part_l, part_acc):
    """Textbook float64 merge of per-slot partial softmaxes (log2 units).

    Unwritten slots carry m = -inf and are excluded even when their l/acc
    hold NaN. Returns `(out [B, S, H, D], lse [B, H, S])`, lse in log2 units.
    """
    m = part_m.to(torch.float64)
    written = m > float("-inf")
    m_g = torch.where(written, m, torch.full_like(m, float("-inf"))).amax(-1)
    w = torch.where(written, torch.exp2(m - m_g[..., None]), torch.zeros_like(m))
    l_i = torch.where(written, part_l.to(torch.float64), torch.zeros_like(m))
    a_i = torch.where(written[..., None], part_acc.to(torch.float64),
                      torch.zeros_like(part_acc, dtype=torch.float64))
    l = (w * l_i).sum(-1)
    acc = (w[..., None] * a_i).sum(-2)
    out = acc / l[..., None]
    lse = m_g + torch.log2(l)
    return out.permute(0, 2, 1, 3), lse
