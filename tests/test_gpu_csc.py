"""The CSC transpose on the GPU against the oracle's reference builder."""

import pytest
import torch

from conftest import make_qkv, oracle_cfg
from moba.config import MoBAConfig
from moba.kernels.routing import build_csc_from_indices, build_csc_fused, csc_to_mask
from oracle import naive as O

pytestmark = pytest.mark.gpu


def column_sets(index, b, kv, blk):
    lo = int(index.col_offsets[b, kv, blk])
    n = int(index.col_nnz[b, kv, blk])
    r = index.row_indices[b, kv, lo:lo + n].tolist()
    h = index.head_indices[b, kv, lo:lo + n].tolist()
    s = index.slot_of_pair[b, kv, lo:lo + n].tolist()
    return sorted(zip(h, r, s))


@pytest.mark.parametrize("b,s,hq,hkv,bs,tk", [(1, 2048, 4, 4, 64, 8), (2, 1024, 4, 2, 32, 4),
                                              (1, 4096, 8, 2, 128, 8), (1, 1000, 2, 1, 128, 5)])
def test_csc_matches_reference_builder(device, b, s, hq, hkv, bs, tk):
    cfg = MoBAConfig(block_size=bs, top_k=tk)
    q, k, _ = make_qkv((b, s, hq, 64), torch.bfloat16, seed=1, device=device)
    k = k[:, :, :hkv].contiguous()
    index = build_csc_fused(q, k, cfg)
    sel = O.moba_selection(q.cpu(), k.cpu(), oracle_cfg(cfg))
    ref = O.build_csc(sel, hkv, tk)
    assert torch.equal(index.col_nnz.cpu(), ref["col_nnz"])
    assert torch.equal(index.col_offsets.cpu(), ref["col_offsets"])
    assert torch.equal(index.order.cpu(), ref["order"]), "longest-first order differs"
    assert torch.equal(csc_to_mask(index, s).cpu(), sel)
    # every entry in place: the build orders a column by (query head, row),
    # as the dense-mask builder does
    for f in ("row_indices", "head_indices", "slot_of_pair"):
        for bi in range(b):
            for kv in range(hkv):
                tot = int(ref["col_offsets"][bi, kv, -1])
                assert torch.equal(getattr(index, f)[bi, kv, :tot].cpu(),
                                   ref[f][bi, kv, :tot]), f
    # column membership as a set of (head, row, slot), including slot numbers
    ic = type(index)(**{f: (getattr(index, f).cpu() if torch.is_tensor(getattr(index, f))
                            else getattr(index, f)) for f in index.__dataclass_fields__})
    for bi in range(b):
        for kv in range(hkv):
            for blk in range(0, index.num_blocks, max(1, index.num_blocks // 7)):
                lo = int(ref["col_offsets"][bi, kv, blk])
                n = int(ref["col_nnz"][bi, kv, blk])
                want = sorted(zip(ref["head_indices"][bi, kv, lo:lo + n].tolist(),
                                  ref["row_indices"][bi, kv, lo:lo + n].tolist(),
                                  ref["slot_of_pair"][bi, kv, lo:lo + n].tolist()))
                assert column_sets(ic, bi, kv, blk) == want


def test_csc_slots_are_dense_and_unique(device):
    cfg = MoBAConfig(block_size=64, top_k=6)
    q, k, _ = make_qkv((1, 2048, 2, 64), torch.bfloat16, seed=2, device=device)
    index = build_csc_fused(q, k, cfg)
    total = int(index.col_offsets[0, 0, -1])
    rows = index.row_indices[0, 0, :total].long().cpu()
    heads = index.head_indices[0, 0, :total].long().cpu()
    slots = index.slot_of_pair[0, 0, :total].long().cpu()
    key = (heads * 2048 + rows) * 8 + slots
    assert key.unique().numel() == total, "a (query, slot) pair appears twice"
    counts = torch.bincount(heads * 2048 + rows, minlength=2 * 2048)
    # slot numbers of one query are exactly 0..count-1
    mx = torch.zeros(2 * 2048, dtype=torch.long).scatter_reduce(0, heads * 2048 + rows, slots,
                                                                 reduce="amax")
    seen = counts > 0
    assert bool(seen.any())
    assert torch.equal((mx + 1)[seen], counts[seen])


def test_csc_packed_rows_are_packed_token_indices(device):
    cfg = MoBAConfig(block_size=16, top_k=3)
    lens = [80, 48, 64, 20]
    cu = torch.tensor([0, 80, 128, 192, 212], dtype=torch.int32)
    q, k, _ = make_qkv((1, 212, 2, 64), torch.bfloat16, seed=5, device=device)
    index = build_csc_fused(q, k, cfg, cu_seqlens=cu.to(device), max_seqlen=80)
    sel = O.moba_selection(q.cpu(), k.cpu(), oracle_cfg(cfg), cu_seqlens=cu)
    assert torch.equal(csc_to_mask(index, 212).cpu(), sel)
    for r, ln in enumerate(lens):
        tot = int(index.col_offsets[r, 0, -1])
        rows = index.row_indices[r, 0, :tot]
        assert int(rows.min()) >= int(cu[r]) and int(rows.max()) < int(cu[r + 1])


def test_csc_unselected_columns_exist(device):
    cfg = MoBAConfig(block_size=64, top_k=2, always_select_current=False)
    q, k, _ = make_qkv((1, 1024, 2, 64), torch.bfloat16, device=device)
    index = build_csc_fused(q, k, cfg)
    assert bool((index.col_nnz == 0).any())
    assert int(index.col_offsets[0, 0, -1]) == int(index.col_nnz[0, 0].sum())


def test_csc_ignores_ids_no_query_can_hold(device):
    """Ids outside [0, n_blocks) -- one past the end, or negative other than
    the -1 padding -- never reach an address: the build ignores them, as if
    they were padding. (The gate never writes them; the guard is for caller
    buffers passed through the C ABI.)"""
    from moba.kernels.gating import gate_select
    from moba.kernels.pooling import pool_blocks

    cfg = MoBAConfig(block_size=64, top_k=4)
    q, k, _ = make_qkv((1, 1024, 2, 64), torch.bfloat16, seed=7, device=device)
    nb = 1024 // 64
    idx = gate_select(q, pool_blocks(k, cfg), cfg)
    g = torch.Generator().manual_seed(3)
    pick = torch.rand(idx.shape, generator=g) < 0.1
    bad = idx.clone()
    bad[pick.to(device) & (torch.arange(4, device=device) % 2 == 0)] = nb
    bad[pick.to(device) & (torch.arange(4, device=device) % 2 == 1)] = -7
    want = build_csc_from_indices(torch.where(pick.to(device), -1, idx), nb, cfg)
    got = build_csc_from_indices(bad, nb, cfg)
    torch.cuda.synchronize()
    assert torch.equal(got.col_nnz, want.col_nnz)
    assert torch.equal(got.col_offsets, want.col_offsets)
    for blk in range(nb):
        assert column_sets(got, 0, 0, blk) == column_sets(want, 0, 0, blk)
        assert column_sets(got, 0, 1, blk) == column_sets(want, 0, 1, blk)


def synthetic_ids(rows, h_q, s, slots, bs_eff, seed, lens=None):
    """Distinct valid ids per query, causal at block size bs_eff (-1 padded
    when a query can see fewer than `slots` blocks)."""
    g = torch.Generator().manual_seed(seed)
    t = torch.arange(s)
    if lens is not None:  # packed: position within the query's own sequence
        starts = torch.repeat_interleave(torch.tensor([0] + lens[:-1]).cumsum(0),
                                         torch.tensor(lens))
        t = t - starts
    vis = (t // bs_eff + 1).view(1, 1, s, 1)
    keys = torch.rand(rows, h_q, s, 4 * slots, generator=g)
    cand = (keys * vis).long()  # in [0, vis)
    idx = torch.full((rows, h_q, s, slots), -1, dtype=torch.long)
    for j in range(4 * slots):  # first `slots` distinct candidates
        c = cand[..., j:j + 1]
        fresh = ~(idx == c).any(-1, keepdim=True)
        free = (idx == -1).int().argmax(-1, keepdim=True)
        room = (idx == -1).any(-1, keepdim=True)
        put = fresh & room
        idx.scatter_(-1, free, torch.where(put, c, idx.gather(-1, free)))
    return idx.to(torch.int32)


def canonical(block_idx, nb, h_kv, cu=None):
    """Per (row, kv head): the (block, head, row, slot) of every entry in
    (block, query head, row) order -- computed with torch sorts."""
    rows, h_q, s, slots = block_idx.shape
    if cu is not None:
        rows = cu.numel() - 1
    g = h_q // h_kv
    out = {}
    for r in range(rows):
        for kv in range(h_kv):
            ids = []
            for hh in range(kv * g, kv * g + g):
                if cu is None:
                    bi = block_idx[r, hh]
                    tok = torch.arange(s)
                else:
                    lo, hi = int(cu[r]), int(cu[r + 1])
                    bi = block_idx[0, hh, lo:hi]
                    tok = torch.arange(lo, hi)
                q, j = (bi >= 0).nonzero(as_tuple=True)
                ids.append(torch.stack([bi[q, j].long(), torch.full_like(q, hh), tok[q], j], 1))
            e = torch.cat(ids)
            key = (e[:, 0] * h_q + e[:, 1]) * (1 << 40) + e[:, 2]
            out[(r, kv)] = e[key.argsort(stable=True)]
    return out


def entries(index, r, kv):
    tot = int(index.col_offsets[r, kv, -1])
    nnz = index.col_nnz[r, kv].long().cpu()
    blk = torch.repeat_interleave(torch.arange(nnz.numel()), nnz)
    return torch.stack([blk, index.head_indices[r, kv, :tot].long().cpu(),
                        index.row_indices[r, kv, :tot].long().cpu(),
                        index.slot_of_pair[r, kv, :tot].long().cpu()], 1)


@pytest.mark.parametrize("s,nb,packed,slots", [(8000, 1000, False, 4), (8000, 1000, True, 4),
                                               (8000, 1000, False, 1),   # rows in halves
                                               (8000, 1000, False, 3),   # queries straddle rows
                                               (6000, 1000, True, 5),
                                               (24000, 12000, False, 4),  # > 64 KiB of LDS
                                               (40000, 20000, False, 4),  # two windows
                                               (60000, 40000, True, 3)])  # three windows
def test_csc_column_order(device, s, nb, packed, slots):
    """The entries of a column come in (query head, row) order, also past
    16384 columns, where the build places the columns window by window."""
    h_q, h_kv = 4, 2
    cfg = MoBAConfig(block_size=64, top_k=slots)
    lens = {8000: [3000, 1000, 4000], 6000: [2500, 1500, 2000],
            60000: [15000, 5000, 40000]}[s] if packed else None
    rps = max(lens) if packed else s
    bs_eff = -(-rps // nb)
    idx = synthetic_ids(1 if packed else 2, h_q, s, slots, bs_eff, seed=11, lens=lens)
    cu = (torch.tensor([0] + lens, dtype=torch.int32).cumsum(0).to(torch.int32)
          if packed else None)
    got = build_csc_from_indices(idx.to(device), nb, cfg, num_kv_heads=h_kv,
                                 cu_seqlens=None if cu is None else cu.to(device),
                                 max_seqlen=rps if packed else None)
    want = canonical(idx, nb, h_kv, cu)
    for (r, kv), w in want.items():
        assert torch.equal(entries(got, r, kv), w), (r, kv)
    # Longest column first, ties by ascending id (routing.py:548-553); above
    # 4096 columns the build sorts, below it ranks.
    nnz = got.col_nnz.long().cpu()
    want_order = torch.argsort(-nnz, dim=-1, stable=True).to(torch.int32)
    assert torch.equal(got.order.cpu(), want_order)


def test_gradients_are_bitwise_stable_across_index_builds(device):
    """Two separately built indexes give the same dQ, dK and dV bit for bit
    (the backward sums a column in its entry order, which is fixed)."""
    from moba.kernels.attention import moba_attention

    cfg = MoBAConfig(block_size=128, top_k=8)
    q, k, v = make_qkv((1, 16384, 4, 64), torch.bfloat16, seed=4, device=device)
    dout = torch.randn_like(q)
    grads = []
    for _ in range(2):
        index = build_csc_fused(q, k, cfg)
        qq, kk, vv = (x.detach().clone().requires_grad_(True) for x in (q, k, v))
        out = moba_attention(qq, kk, vv, cfg, index=index)
        out.backward(dout)
        grads.append((out.detach(), qq.grad, kk.grad, vv.grad))
    for a, b in zip(*grads):
        assert torch.equal(a, b)
