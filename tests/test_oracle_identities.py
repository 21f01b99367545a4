"""Exact identities the mathematics fixes, run on the oracle in float64.

These pin the oracle where no reference vector reaches (reference
`tests/test_semantics.py` Tier 1), chosen so a dropped term, a wrong index or
a flipped sign fails one of them: closed-form block means, brute-force
selection on tiny inputs, reduction to dense causal attention, single-block
causal attention, the gather form against the dense form, the textbook merge
against a direct softmax, and the CSC round trip.
"""

import itertools
import math

import pytest
import torch
import torch.nn.functional as F

from conftest import oracle_cfg
from oracle import c_oracle
from oracle import naive as O


def cfg(bs, tk, **kw):
    from moba.config import MoBAConfig
    return oracle_cfg(MoBAConfig(block_size=bs, top_k=tk, **kw))


def qkv(b, s, h, d, dtype=torch.float64, seed=0):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(b, s, h, d, generator=g, dtype=dtype) for _ in range(3))


@pytest.mark.parametrize("s,bs", [(128, 32), (129, 32), (64, 64), (100, 16)])
def test_pool_is_block_mean_with_real_tail_count(s, bs):
    _, k, _ = qkv(1, s, 2, 16)
    kbar = O.pool_blocks(k, bs)
    n = math.ceil(s / bs)
    assert kbar.shape == (1, 2, n, 16)
    for j in range(n):
        torch.testing.assert_close(kbar[:, :, j], k[:, j * bs:(j + 1) * bs].mean(dim=1),
                                   rtol=0, atol=1e-14)


def brute_force_selection(q, kbar, c):
    """Enumerates every candidate per query and sorts (score desc, id asc)."""
    b, s, h, _ = q.shape
    n = kbar.shape[2]
    take = O.past_blocks_selected(c, n)
    kb = O.expand_kv(kbar, h, dim=1)
    out = torch.zeros(b, h, s, n, dtype=torch.bool)
    for bi, hi, t in itertools.product(range(b), range(h), range(s)):
        own = t // c.block_size
        cands = []
        for j in range(own):
            sc = float(torch.dot(q[bi, t, hi].double(), kb[bi, hi, j].double()))
            cands.append((-sc, j))
        cands.sort()
        for _, j in cands[:take]:
            out[bi, hi, t, j] = True
        if c.always_select_current:
            out[bi, hi, t, own] = True
    return out


@pytest.mark.parametrize("s,bs,tk,h,hkv", [(96, 8, 3, 2, 2), (77, 8, 4, 4, 2), (64, 16, 2, 1, 1)])
def test_gate_equals_brute_force(s, bs, tk, h, hkv):
    q, k, _ = qkv(1, s, h, 8)
    k = k[:, :, :hkv].contiguous()
    c = cfg(bs, tk)
    kbar = O.pool_blocks(k, bs)
    assert torch.equal(O.gate_select(q, kbar, c), brute_force_selection(q, kbar, c))


def test_ties_go_to_the_lower_block_in_both_oracles():
    q, k, _ = qkv(1, 512, 1, 64, dtype=torch.bfloat16)
    c = cfg(64, 3)
    kbar = O.pool_blocks(k, 64)
    kbar[:] = kbar[:, :, :1]
    idx = O.mask_to_indices(O.gate_select(q, kbar, c), 3)
    late = idx[0, 0, 400]
    assert late.tolist() == [0, 1, 6]
    assert torch.equal(c_oracle.gate_select(q, kbar, c), idx)


def test_selection_structure():
    q, k, _ = qkv(1, 1024, 2, 32, dtype=torch.bfloat16, seed=3)
    c = cfg(32, 5)
    sel = O.moba_selection(q, k, c)
    own = torch.arange(1024) // 32
    blocks = torch.arange(sel.shape[-1])
    assert bool(sel[..., torch.arange(1024), own].all()), "own block not selected"
    future = blocks.view(1, -1) > own.view(-1, 1)
    assert not bool((sel & future).any()), "a future block was selected"
    assert int(sel.sum(-1).max()) == 5
    assert torch.equal(sel.sum(-1)[0, 0, :32], torch.ones(32, dtype=torch.int64))


def test_reduces_to_dense_causal_attention_when_every_block_fits():
    q, k, v = qkv(1, 256, 2, 32)
    c = cfg(32, 8)  # 8 blocks, top_k 8: everything selected
    o = O.moba_attention(q, k, v, c)
    ref = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2),
                                         v.transpose(1, 2), is_causal=True).transpose(1, 2)
    torch.testing.assert_close(o, ref, rtol=0, atol=1e-12)


def test_single_block_is_causal_attention_and_first_query_sees_itself():
    q, k, v = qkv(1, 64, 2, 16)
    o = O.moba_attention(q, k, v, cfg(64, 1))
    ref = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2),
                                         v.transpose(1, 2), is_causal=True).transpose(1, 2)
    torch.testing.assert_close(o, ref, rtol=0, atol=1e-12)
    torch.testing.assert_close(o[:, 0], v[:, 0], rtol=0, atol=1e-14)


def test_query_chunking_is_bitwise_identical():
    q, k, v = qkv(1, 300, 2, 16, seed=4)
    c = cfg(32, 3)
    assert torch.equal(O.moba_attention(q, k, v, c), O.moba_attention(q, k, v, c, query_chunk=64))


@pytest.mark.parametrize("h,hkv", [(2, 2), (4, 2)])
def test_sparse_gather_form_equals_dense_form(h, hkv):
    q, k, v = qkv(1, 333, h, 16, seed=5)
    k, v = k[:, :, :hkv].contiguous(), v[:, :, :hkv].contiguous()
    c = cfg(32, 4)
    sel = O.moba_selection(q, k, c)
    dense = O.moba_attention(q, k, v, c, selected=sel)
    idx = O.mask_to_indices(sel, 4)
    sparse, lse = O.moba_attention_sparse(q, k, v, idx, 32)
    torch.testing.assert_close(sparse, dense, rtol=0, atol=1e-12)
    rows = torch.tensor([0, 17, 200, 332])
    part, _ = O.moba_attention_sparse(q, k, v, idx, 32, rows=rows)
    torch.testing.assert_close(part, dense[:, rows], rtol=0, atol=1e-12)


def test_textbook_merge_equals_direct_softmax():
    """Split a row's logits into slots, form (m, l, acc) per slot in log2
    units, merge: the result must equal softmax over the whole row."""
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(3, 5, 40, generator=g, dtype=torch.float64) * 3
    vals = torch.randn(3, 5, 40, 8, generator=g, dtype=torch.float64)
    lg2 = logits * math.log2(math.e)
    slots = 4
    part_m = torch.empty(1, 3, 5, slots, dtype=torch.float64)
    part_l = torch.empty_like(part_m)
    part_acc = torch.empty(1, 3, 5, slots, 8, dtype=torch.float64)
    for j in range(slots):
        seg = slice(j * 10, (j + 1) * 10)
        m = lg2[..., seg].amax(-1)
        p = torch.exp2(lg2[..., seg] - m[..., None])
        part_m[0, ..., j] = m
        part_l[0, ..., j] = p.sum(-1)
        part_acc[0, ..., j, :] = (p[..., None] * vals[..., seg, :]).sum(-2)
    out, lse = O.combine_reference(part_m, part_l, part_acc)
    ref = (torch.softmax(logits, -1)[..., None] * vals).sum(-2)
    torch.testing.assert_close(out[0].transpose(0, 1), ref, rtol=0, atol=1e-12)
    torch.testing.assert_close(lse[0], torch.logsumexp(logits, -1) * math.log2(math.e),
                               rtol=0, atol=1e-12)
    # An unwritten slot (m = -inf) holding NaN is ignored.
    part_m[0, 0, 0, 1] = float("-inf")
    part_acc[0, 0, 0, 1] = float("nan")
    part_l[0, 0, 0, 1] = float("nan")
    out2, _ = O.combine_reference(part_m, part_l, part_acc)
    assert bool(torch.isfinite(out2).all())


def test_csc_round_trips_and_is_consistent():
    q, k, _ = qkv(1, 512, 4, 32, dtype=torch.bfloat16, seed=6)
    k = k[:, :, :2].contiguous()
    c = cfg(32, 4)
    sel = O.moba_selection(q, k, c)
    idx = O.build_csc(sel, 2, 4)
    back = O.csc_to_mask(idx["col_nnz"], idx["col_offsets"], idx["row_indices"],
                         idx["head_indices"], 4, 512)
    assert torch.equal(back, sel)
    counts = idx["col_nnz"].long()
    order = idx["order"].long()
    sc = counts.gather(-1, order)
    assert bool((sc[..., 1:] <= sc[..., :-1]).all())
    ties = sc[..., 1:] == sc[..., :-1]
    assert bool(((order[..., 1:] > order[..., :-1]) | ~ties).all())


def test_slot_numbering_is_rank_by_ascending_block():
    q, k, _ = qkv(1, 256, 2, 32, dtype=torch.bfloat16, seed=7)
    c = cfg(32, 3)
    sel = O.moba_selection(q, k, c)
    idx = O.mask_to_indices(sel, 3)
    valid = idx >= 0
    both = valid[..., 1:] & valid[..., :-1]
    assert bool(((idx[..., 1:] > idx[..., :-1]) | ~both).all())
    assert bool((valid[..., 1:] <= valid[..., :-1]).all())
    assert torch.equal(O.indices_to_mask(idx, sel.shape[-1]), sel)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
def test_c_oracle_equals_torch_oracle(dt):
    q, k, _ = qkv(2, 700, 4, 64, dtype=dt, seed=8)
    k = k[:, :, :2].contiguous()
    c = cfg(64, 5)
    kb = O.pool_blocks(k, 64)
    assert torch.equal(c_oracle.pool_blocks(k, 64), kb)
    assert torch.equal(c_oracle.gate_select(q, kb, c),
                       O.mask_to_indices(O.gate_select(q, kb, c), 5))


@pytest.mark.parametrize("heads,off,stride", [(range(0, 4), 0, 1), (range(1, 3), 3, 8),
                                              (range(3, 4), 5, 7)])
def test_strided_c_gate_equals_the_torch_gate_restricted(heads, off, stride):
    """The C oracle's head / row subset (used on whole heads at 512K) is the
    torch oracle's full gate read at those heads and rows, for two batch
    rows, GQA and a ragged tail."""
    c = cfg(64, 6)
    q, k, _ = (t.to(torch.bfloat16) for t in qkv(2, 1000, 4, 64, dtype=torch.float32, seed=12))
    kbar = O.pool_blocks(k[:, :, :2].contiguous(), 64)
    full = O.mask_to_indices(O.gate_select(q, kbar, c), 6)
    got = c_oracle.gate_select_strided(q, kbar, c, heads=heads, offset=off, stride=stride)
    assert torch.equal(got, full[:, heads.start:heads.stop, off::stride])


@pytest.mark.parametrize("s,bs,tk", [(2048, 64, 5), (1000, 32, 8)])
def test_gate_rows_equal_the_full_gate_restricted(s, bs, tk):
    """The row-subset gate (used at full sequence lengths) is the full gate
    read at those rows, including the first rows, block edges and the tail."""
    c = cfg(bs, tk)
    q, k, _ = (t.to(torch.bfloat16) for t in qkv(2, s, 4, 64, dtype=torch.float32, seed=9))
    kbar = O.pool_blocks(k, bs)
    full = O.gate_select(q, kbar, c)
    rows = torch.tensor(sorted({0, 1, bs - 1, bs, 3 * bs + 7, s // 2, s - 2, s - 1}))
    assert torch.equal(O.gate_select_rows(q, kbar, c, rows), full[:, :, rows])


@pytest.mark.parametrize("s,bs,tk", [(1000, 64, 4), (1024, 128, 8), (777, 32, 3), (256, 128, 8)])
def test_sparsity_ratio_counts_the_selected_keys(s, bs, tk):
    """The closed form behind the attainment ceiling equals the attended-key
    count of real selections (the oracle gate on random inputs): own block's
    causal prefix plus every key of each selected past block, over all
    causally legal keys (reference `tests/test_bench.py` cross-check)."""
    from moba.config import MoBAConfig
    from moba.sparsity import sparsity_ratio

    q, k, _ = qkv(1, s, 2, 32, dtype=torch.float32, seed=5)
    sel = O.moba_selection(q, k, cfg(bs, tk))                    # [1, H, S, nb]
    i = torch.arange(s)
    key_block = torch.arange(s) // bs
    visible = sel[..., key_block] & (torch.arange(s).view(1, -1) <= i.view(-1, 1))
    attended = visible.sum(dtype=torch.float64) / sel.shape[1]
    want = attended / (i + 1).sum(dtype=torch.float64)
    got = sparsity_ratio(s, MoBAConfig(block_size=bs, top_k=tk))
    assert abs(got - want.item()) < 1e-12


@pytest.mark.parametrize("h,hkv", [(2, 2), (4, 2)])
def test_hand_gradients_equal_autograd_of_the_dense_form(h, hkv):
    """`sparse_grads` (the explicit backward used at full sizes) against torch
    autograd of the dense oracle: all rows and keys, then a row subset with
    dK / dV restricted to some blocks."""
    q, k, v = qkv(1, 333, h, 16, seed=6)
    k, v = k[:, :, :hkv].contiguous(), v[:, :, :hkv].contiguous()
    do = qkv(1, 333, h, 16, seed=7)[0]
    c = cfg(32, 4)
    sel = O.moba_selection(q, k, c)
    idx = O.mask_to_indices(sel, 4)
    lq, lk, lv = (t.clone().requires_grad_(True) for t in (q, k, v))
    ref = O.moba_attention(lq, lk, lv, c, selected=sel)
    ref.backward(do)
    out, dq, dk, dv = O.sparse_grads(q, k, v, do, idx, 32, torch.arange(333))
    for got, want in ((out, ref.detach()), (dq, lq.grad), (dk, lk.grad), (dv, lv.grad)):
        torch.testing.assert_close(got, want, rtol=0, atol=1e-12)
    # A row subset: out and dq of those rows; dk / dv of blocks {0, 5} from
    # every row that selected them equal autograd's on those keys.
    rows = torch.tensor([0, 40, 200, 332])
    out, dq, _, _ = O.sparse_grads(q, k, v, do, idx, 32, rows, max_gather_bytes=1 << 14)
    torch.testing.assert_close(out, ref.detach()[:, rows], rtol=0, atol=1e-12)
    torch.testing.assert_close(dq, lq.grad[:, rows], rtol=0, atol=1e-12)
    users = torch.nonzero((idx[..., None] == torch.tensor([0, 5])).any(-1).any(-1).any(1)[0])
    keys = torch.cat([torch.arange(0, 32), torch.arange(160, 192)])
    for only in (False, True):
        _, _, dk, dv = O.sparse_grads(q, k, v, do, idx, 32, users.flatten(), key_blocks=[0, 5],
                                      key_users_only=only)
        torch.testing.assert_close(dk[:, keys], lk.grad[:, keys], rtol=0, atol=1e-12)
        torch.testing.assert_close(dv[:, keys], lv.grad[:, keys], rtol=0, atol=1e-12)
        assert not bool(dk[:, 32:160].any()), "keys outside key_blocks must stay zero"


def test_hand_gradients_in_bfloat16_track_float64():
    """The same-dtype oracle: bfloat16 products, one rounding per sum. Its
    error against float64 is of bfloat16 size, neither zero nor large."""
    q, k, v = qkv(1, 256, 2, 64, seed=8)
    do = qkv(1, 256, 2, 64, seed=9)[0]
    q, k, v, do = (t.bfloat16().double() for t in (q, k, v, do))
    idx = O.mask_to_indices(O.moba_selection(q, k, cfg(32, 4)), 4)
    rows = torch.arange(256)
    hi = O.sparse_grads(q, k, v, do, idx, 32, rows)
    lo = O.sparse_grads(q, k, v, do, idx, 32, rows, dtype=torch.bfloat16)
    for a, b in zip(lo, hi):
        assert a.dtype is torch.bfloat16
        err = (a.double() - b).abs().max().item()
        assert 1e-5 < err < 5e-2 * max(1.0, b.abs().max().item()), err


def _brute_hierarchical(q, k, bs, tk, group, opened):
    """Per query, in plain loops: super-block scores of the representatives'
    means, the best `opened` past super-blocks, then the best past blocks
    inside them (and inside the own super-block) by (score desc, id asc)."""
    b, s, h, d = q.shape
    kbar = O.pool_blocks(k, bs)
    n = kbar.shape[2]
    sbar = O.super_block_means(kbar, group)
    take = min(tk - 1, n)
    out = torch.zeros(b, h, s, n, dtype=torch.bool)
    for bi in range(b):
        for hi in range(h):
            for t in range(s):
                own = t // bs
                own_sb = t // (bs * group)
                sups = sorted(range(own_sb), key=lambda x: (-float(O.round_to_dtype(
                    (q[bi, t, hi].double() * sbar[bi, hi, x].double()).sum(), q.dtype)), x))
                opened_set = set(sups[:opened]) | {own_sb}
                cands = [j for j in range(own) if j // group in opened_set]
                ranked = sorted(cands, key=lambda j: (-float(O.round_to_dtype(
                    (q[bi, t, hi].double() * kbar[bi, hi, j].double()).sum(), q.dtype)), j))
                for j in ranked[:take]:
                    out[bi, hi, t, j] = True
                out[bi, hi, t, own] = True
    return out


@pytest.mark.parametrize("s,bs,tk,group,opened", [(256, 8, 4, 4, 2), (300, 16, 3, 2, 1),
                                                 (512, 8, 5, 8, 3)])
def test_hierarchical_gate_equals_brute_force(s, bs, tk, group, opened):
    q, k, _ = qkv(1, s, 2, 16, seed=12)
    c = cfg(bs, tk)
    got = O.hierarchical_select(q, O.pool_blocks(k, bs), c, group, opened)
    assert torch.equal(got, _brute_hierarchical(q, k, bs, tk, group, opened))


@pytest.mark.parametrize("dt", [torch.float64, torch.bfloat16])
def test_hierarchical_gate_reduces_to_the_exact_gate(dt):
    """Opening every super-block, or super-blocks of one block opened as many
    as the past budget, leaves the exact gate."""
    q, k, _ = qkv(1, 1024, 2, 32, seed=13)
    q, k = q.to(dt), k.to(dt)
    c = cfg(16, 6)
    kbar = O.pool_blocks(k, 16)
    exact = O.gate_select(q, kbar, c)
    assert torch.equal(O.hierarchical_select(q, kbar, c, 4, 1024 // 64), exact)
    assert torch.equal(O.hierarchical_select(q, kbar, c, 1, 5), exact)
    # A real restriction changes some selections and never the own block.
    h = O.hierarchical_select(q, kbar, c, 4, 1)
    assert not torch.equal(h, exact)
    own = (torch.arange(1024) // 16)
    assert bool(h[0, :, torch.arange(1024), own].all())
    assert int(h.sum(-1).max()) <= 6


def test_hierarchical_gate_rows_equal_the_full_result_restricted():
    q, k, _ = qkv(1, 700, 2, 16, seed=14)
    c = cfg(16, 4)
    kbar = O.pool_blocks(k, 16)
    rows = torch.tensor([0, 15, 16, 200, 511, 699])
    full = O.hierarchical_select(q, kbar, c, 4, 2)
    assert torch.equal(O.hierarchical_select(q, kbar, c, 4, 2, rows=rows), full[:, :, rows])
