"""Forward, merge and backward on the GPU against the fp64 oracle."""

import math

import pytest
import torch

from conftest import make_qkv, oracle_cfg
from gpu_util import fp64_truth, oracle_selection, to_cpu
from moba.config import MoBAConfig
from moba.kernels.attention import moba_attention
from moba.kernels.moba_fwd import combine_partials, moba_forward
from moba.kernels.routing import build_csc_fused, csc_to_mask
from oracle import naive as O
from tolerance import (BF16_MAX_ABS, BF16_MEAN_ABS, FP32_MAX_ABS, assert_selection_matches,
                       assert_within_tolerance, max_abs_error, mean_abs_error)

pytestmark = pytest.mark.gpu

FWD_CASES = [
    # (shape, h_kv, block_size, top_k)
    ((1, 1024, 4, 128), 4, 64, 8),
    ((2, 1024, 4, 64), 4, 32, 4),
    ((1, 2048, 4, 64), 4, 128, 8),
    ((1, 1000, 2, 64), 2, 128, 5),
    ((1, 2048, 8, 128), 2, 64, 4),
    ((1, 1024, 4, 64), 1, 64, 3),
]


@pytest.mark.parametrize("shape,h_kv,bs,tk", FWD_CASES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_forward_within_tolerance(device, shape, h_kv, bs, tk, dtype):
    cfg = MoBAConfig(block_size=bs, top_k=tk, dtype=dtype)
    q, k, v = make_qkv(shape, dtype, seed=1, device=device)
    k, v = k[:, :, :h_kv].contiguous(), v[:, :, :h_kv].contiguous()
    index = build_csc_fused(q, k, cfg)
    sel = oracle_selection(q, k, cfg)
    assert_selection_matches(csc_to_mask(index, shape[1]), sel, "ours")
    out = moba_forward(q, k, v, cfg, index=index)
    truth, ref_err = fp64_truth(q, k, v, cfg, sel)
    assert_within_tolerance(out, truth, ref_err, "ours")
    if dtype == torch.bfloat16:
        assert max_abs_error(out, truth) <= BF16_MAX_ABS
        assert mean_abs_error(out, truth) <= BF16_MEAN_ABS


@pytest.mark.parametrize("shape,h_kv,bs,tk", [((1, 1024, 4, 64), 4, 64, 8),
                                              ((1, 1024, 4, 128), 2, 128, 4),
                                              ((1, 4096, 4, 64), 4, 128, 8)])
def test_forward_fp32_matches_oracle(device, shape, h_kv, bs, tk):
    cfg = MoBAConfig(block_size=bs, top_k=tk, dtype=torch.float32)
    q, k, v = make_qkv(shape, torch.float32, seed=2, device=device)
    k, v = k[:, :, :h_kv].contiguous(), v[:, :, :h_kv].contiguous()
    out = moba_forward(q, k, v, cfg)
    sel = oracle_selection(q, k, cfg)
    truth, _ = fp64_truth(q, k, v, cfg, sel)
    assert max_abs_error(out, truth) <= FP32_MAX_ABS


def test_forward_packed_equals_each_sequence_alone(device):
    cfg = MoBAConfig(block_size=16, top_k=3)
    lens = [80, 48, 64, 20]
    cu = torch.tensor([0, 80, 128, 192, 212], dtype=torch.int32, device=device)
    q, k, v = make_qkv((1, 212, 2, 64), torch.bfloat16, seed=5, device=device)
    packed = moba_forward(q, k, v, cfg, cu_seqlens=cu, max_seqlen=80)
    for r, ln in enumerate(lens):
        lo = int(cu[r])
        alone = moba_forward(q[:, lo:lo + ln], k[:, lo:lo + ln], v[:, lo:lo + ln], cfg)
        assert torch.equal(packed[:, lo:lo + ln], alone), f"sequence {r}"
    sel = oracle_selection(q, k, cfg, cu_seqlens=cu)
    truth, ref_err = fp64_truth(q, k, v, cfg, sel, cu_seqlens=cu)
    assert_within_tolerance(packed, truth, ref_err, "packed")


def test_forward_is_deterministic_and_routing_fixed_by_index(device):
    cfg = MoBAConfig(block_size=64, top_k=4)
    q, k, v = make_qkv((1, 2048, 2, 64), torch.bfloat16, seed=7, device=device)
    index = build_csc_fused(q, k, cfg)
    a = moba_forward(q, k, v, cfg, index=index)
    b = moba_forward(q, k, v, cfg, index=index)
    assert torch.equal(a, b)
    c = moba_forward(q, k, v, cfg)
    assert torch.equal(a, c), "forward depends on column order"


def reference_combine_inputs(device, b=1, h=2, s=33, slots=5, d=64, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(0)
    m = torch.randn(b, h, s, slots, generator=g) * 4
    l = torch.rand(b, h, s, slots, generator=g) * 3 + 0.5
    acc = torch.randn(b, h, s, slots, d, generator=g)
    return m, l, acc


@pytest.mark.parametrize("slots", [1, 3, 5, 8, 12])
def test_combine_matches_textbook_merge(device, slots):
    m, l, acc = reference_combine_inputs(device, slots=slots)
    acc_b = acc.to(torch.bfloat16)
    out, lse = combine_partials(m.to(device), l.to(device), acc_b.to(device), torch.float32,
                                return_lse=True)
    ref_out, ref_lse = O.combine_reference(m.double(), l.double(), acc_b.double())
    assert max_abs_error(out, ref_out) < 1e-5
    assert max_abs_error(lse, ref_lse) < 1e-5


def test_combine_ignores_unwritten_slots_holding_nan(device):
    m, l, acc = reference_combine_inputs(device, slots=4)
    m[..., 2] = float("-inf")
    l[..., 2] = float("nan")
    acc[..., 2, :] = float("nan")
    out = combine_partials(m.to(device), l.to(device), acc.to(device), torch.float32)
    assert bool(torch.isfinite(out).all())
    ref, _ = O.combine_reference(m.double(), l.double(), acc.double())
    assert max_abs_error(out, ref) < 1e-5


def test_combine_shift_invariance_and_dominant_slot(device):
    m, l, acc = reference_combine_inputs(device, slots=4, dtype=torch.float32)
    out1 = combine_partials(m.to(device), l.to(device), acc.to(device), torch.float32)
    out2 = combine_partials((m + 37.0).to(device), l.to(device), acc.to(device), torch.float32)
    assert max_abs_error(out1, out2) < 1e-5
    m2 = m.clone()
    m2[..., 0] = 500.0
    out3 = combine_partials(m2.to(device), l.to(device), acc.to(device), torch.float32)
    ref = (acc[..., 0, :] / l[..., 0:1]).permute(0, 2, 1, 3)
    assert max_abs_error(out3, ref) < 1e-5


def grads_oracle(q, k, v, cfg, sel, g, dtype=torch.float64):
    qc, kc, vc, gc = (t.detach().cpu().to(dtype).requires_grad_(True) for t in (q, k, v, g))
    out = O.moba_attention(qc, kc, vc, oracle_cfg(cfg), selected=sel, query_chunk=256)
    out.backward(gc.detach())
    return qc.grad, kc.grad, vc.grad


BWD_CASES = [((1, 512, 2, 64), 2, 64, 4), ((1, 1024, 2, 128), 2, 128, 4),
             ((1, 1024, 4, 64), 2, 64, 3), ((2, 640, 2, 64), 2, 32, 6)]


@pytest.mark.parametrize("shape,h_kv,bs,tk", BWD_CASES)
def test_backward_within_tolerance(device, shape, h_kv, bs, tk):
    cfg = MoBAConfig(block_size=bs, top_k=tk)
    q, k, v = make_qkv(shape, torch.bfloat16, seed=3, device=device)
    k, v = k[:, :, :h_kv].contiguous(), v[:, :, :h_kv].contiguous()
    g = make_qkv(shape, torch.bfloat16, seed=4, device=device, n=1)[0]
    sel = oracle_selection(q, k, cfg)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = moba_attention(qq, kk, vv, cfg)
    out.backward(g)
    truth = grads_oracle(q, k, v, cfg, sel, g)
    low = grads_oracle(q, k, v, cfg, sel, g, dtype=torch.bfloat16)
    for name, ours, ref, tr in [("dq", qq.grad, low[0], truth[0]), ("dk", kk.grad, low[1], truth[1]),
                                ("dv", vv.grad, low[2], truth[2])]:
        ref_err = max_abs_error(ref, tr)
        assert_within_tolerance(ours, tr, ref_err, name)
        assert max_abs_error(ours, tr) <= BF16_MAX_ABS, name
        assert mean_abs_error(ours, tr) <= BF16_MEAN_ABS, name


@pytest.mark.parametrize("shape,h_kv,bs,tk", [((1, 1024, 4, 64), 2, 64, 3),
                                             ((1, 1024, 2, 128), 2, 128, 4)])
def test_backward_fp16_within_tolerance(device, shape, h_kv, bs, tk):
    """The float16 backward (same kernels, float16 operands and partials)
    against the float64 oracle, with the oracle's own float16 error as the
    yardstick."""
    cfg = MoBAConfig(block_size=bs, top_k=tk)
    q, k, v = make_qkv(shape, torch.float16, seed=13, device=device)
    k, v = k[:, :, :h_kv].contiguous(), v[:, :, :h_kv].contiguous()
    g = make_qkv(shape, torch.float16, seed=14, device=device, n=1)[0]
    sel = oracle_selection(q, k, cfg)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = moba_attention(qq, kk, vv, cfg)
    out.backward(g)
    truth = grads_oracle(q, k, v, cfg, sel, g)
    low = grads_oracle(q, k, v, cfg, sel, g, dtype=torch.float16)
    for name, ours, ref, tr in [("dq", qq.grad, low[0], truth[0]), ("dk", kk.grad, low[1], truth[1]),
                                ("dv", vv.grad, low[2], truth[2])]:
        assert_within_tolerance(ours, tr, max_abs_error(ref, tr), name)
        assert max_abs_error(ours, tr) <= BF16_MAX_ABS, name
        assert mean_abs_error(ours, tr) <= BF16_MEAN_ABS, name


def test_backward_fp32_matches_autograd(device):
    cfg = MoBAConfig(block_size=64, top_k=4, dtype=torch.float32)
    shape = (1, 512, 2, 64)
    q, k, v = make_qkv(shape, torch.float32, seed=3, device=device)
    g = make_qkv(shape, torch.float32, seed=4, device=device, n=1)[0]
    sel = oracle_selection(q, k, cfg)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    moba_attention(qq, kk, vv, cfg).backward(g)
    truth = grads_oracle(q, k, v, cfg, sel, g)
    for ours, tr in zip((qq.grad, kk.grad, vv.grad), truth):
        assert max_abs_error(ours, tr) <= FP32_MAX_ABS


@pytest.mark.parametrize("shape,h_kv,bs,tk", [((1, 1024, 8, 64), 2, 128, 4),
                                              ((1, 2048, 4, 64), 4, 128, 8),
                                              ((1, 1024, 4, 128), 1, 64, 3)])
def test_backward_fp32_gqa_and_bs128_match_autograd(device, shape, h_kv, bs, tk):
    """The float32 path at 1e-5: GQA groups of 4 and 8 query heads per kv
    head, D 128, and the headline's block size 128 / top-k 8."""
    cfg = MoBAConfig(block_size=bs, top_k=tk, dtype=torch.float32)
    q, k, v = make_qkv(shape, torch.float32, seed=23, device=device)
    k, v = k[:, :, :h_kv].contiguous(), v[:, :, :h_kv].contiguous()
    g = make_qkv(shape, torch.float32, seed=24, device=device, n=1)[0]
    sel = oracle_selection(q, k, cfg)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = moba_attention(qq, kk, vv, cfg)
    out.backward(g)
    qc, kc, vc, gc = (t.detach().cpu().double().requires_grad_(True) for t in (q, k, v, g))
    ref = O.moba_attention(qc, kc, vc, oracle_cfg(cfg), selected=sel, query_chunk=256)
    ref.backward(gc.detach())
    for name, ours, tr in (("out", out, ref), ("dq", qq.grad, qc.grad), ("dk", kk.grad, kc.grad),
                           ("dv", vv.grad, vc.grad)):
        assert max_abs_error(ours, tr) <= FP32_MAX_ABS, name


def test_backward_fp32_packed_matches_autograd(device):
    cfg = MoBAConfig(block_size=64, top_k=4, dtype=torch.float32)
    lens = [500, 128, 700]
    cu = torch.tensor([0, 500, 628, 1328], dtype=torch.int32, device=device)
    q = make_qkv((1, 1328, 4, 64), torch.float32, seed=25, device=device, n=1)[0]
    k, v = make_qkv((1, 1328, 2, 64), torch.float32, seed=26, device=device, n=2)
    g = make_qkv((1, 1328, 4, 64), torch.float32, seed=27, device=device, n=1)[0]
    sel = oracle_selection(q, k, cfg, cu_seqlens=cu)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = moba_attention(qq, kk, vv, cfg, cu_seqlens=cu, max_seqlen=max(lens))
    out.backward(g)
    qc, kc, vc, gc = (t.detach().cpu().double().requires_grad_(True) for t in (q, k, v, g))
    ref = O.moba_attention(qc, kc, vc, oracle_cfg(cfg), selected=sel, cu_seqlens=cu.cpu())
    ref.backward(gc.detach())
    for name, ours, tr in (("out", out, ref), ("dq", qq.grad, qc.grad), ("dk", kk.grad, kc.grad),
                           ("dv", vv.grad, vc.grad)):
        assert max_abs_error(ours, tr) <= FP32_MAX_ABS, name


def test_unselected_blocks_get_exactly_zero_gradient(device):
    cfg = MoBAConfig(block_size=64, top_k=2, always_select_current=False)
    shape = (1, 1024, 2, 64)
    q, k, v = make_qkv(shape, torch.bfloat16, device=device)
    g = make_qkv(shape, torch.bfloat16, seed=9, device=device, n=1)[0] * 0.1
    index = build_csc_fused(q, k, cfg)
    empty = index.col_nnz == 0
    assert bool(empty.any())
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = moba_attention(qq, kk, vv, cfg, index=index)
    out = torch.nan_to_num(out)  # queries with no selection produce NaN by design
    out.backward(g)
    for b, h, blk in empty.nonzero().tolist():
        lo, hi = blk * 64, min(blk * 64 + 64, 1024)
        assert not bool(kk.grad[b, lo:hi, h].any())
        assert not bool(vv.grad[b, lo:hi, h].any())


def test_backward_is_deterministic_given_an_index(device):
    cfg = MoBAConfig(block_size=64, top_k=4)
    shape = (1, 1024, 2, 64)
    q, k, v = make_qkv(shape, torch.bfloat16, seed=11, device=device)
    g = make_qkv(shape, torch.bfloat16, seed=12, device=device, n=1)[0]
    index = build_csc_fused(q, k, cfg)
    res = []
    for _ in range(2):
        qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
        moba_attention(qq, kk, vv, cfg, index=index).backward(g)
        res.append((qq.grad, kk.grad, vv.grad))
    for a, b in zip(*res):
        assert torch.equal(a, b)


def test_packed_backward_equals_each_sequence_alone(device):
    cfg = MoBAConfig(block_size=16, top_k=3)
    lens = [80, 48, 64, 20]
    cu = torch.tensor([0, 80, 128, 192, 212], dtype=torch.int32, device=device)
    q, k, v = make_qkv((1, 212, 2, 64), torch.bfloat16, seed=5, device=device)
    g = make_qkv((1, 212, 2, 64), torch.bfloat16, seed=6, device=device, n=1)[0]
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    moba_attention(qq, kk, vv, cfg, cu_seqlens=cu, max_seqlen=80).backward(g)
    for r, ln in enumerate(lens):
        lo = int(cu[r])
        a = [t[:, lo:lo + ln].clone().requires_grad_(True) for t in (q, k, v)]
        moba_attention(*a, cfg).backward(g[:, lo:lo + ln])
        # dq is per query and exact; dk / dv sum down a column whose entry
        # order is unspecified, so they may differ in the last bf16 bit.
        assert torch.equal(qq.grad[:, lo:lo + ln], a[0].grad), f"dq, sequence {r}"
        for ours, alone in zip((kk.grad, vv.grad), a[1:]):
            assert max_abs_error(ours[:, lo:lo + ln], alone.grad) < 2e-2, f"sequence {r}"


@pytest.mark.parametrize("shape,h_kv", [((1, 1024, 4, 64), 4), ((2, 512, 8, 128), 2)])
def test_every_block_selected_matches_dense_sdpa(device, shape, h_kv):
    """top_k >= blocks: MoBA is dense causal attention, so the HIP forward
    must agree with torch's fused SDPA (the `sdpa_dense` baseline backend)
    within the bf16 bars -- a cross-check independent of the oracle."""
    from implementations import get_backend

    q, k, v = make_qkv(shape, torch.bfloat16, seed=11)
    k, v = k[:, :, :h_kv].contiguous(), v[:, :, :h_kv].contiguous()
    cfg = MoBAConfig(block_size=128, top_k=shape[1] // 128)
    qg, kg, vg = (t.to(device) for t in (q, k, v))
    ours = moba_forward(qg, kg, vg, cfg).float()
    dense = get_backend("sdpa_dense").forward(qg, kg, vg, cfg).float()
    assert max_abs_error(ours, dense) <= BF16_MAX_ABS
    assert mean_abs_error(ours, dense) <= BF16_MEAN_ABS


def test_sdpa_dense_packed_equals_each_sequence_alone(device):
    from implementations import get_backend

    be = get_backend("sdpa_dense")
    lens = [384, 128, 640]
    cu = torch.tensor([0, 384, 512, 1152], dtype=torch.int32, device=device)
    q, k, v = (t.to(device) for t in make_qkv((1, sum(lens), 4, 64), torch.bfloat16, seed=2))
    cfg = MoBAConfig(block_size=128, top_k=8)
    packed = be.forward_packed(q, k, v, cfg, cu)
    for lo, hi in zip(cu.tolist()[:-1], cu.tolist()[1:]):
        alone = be.forward(q[:, lo:hi], k[:, lo:hi], v[:, lo:hi], cfg)
        assert torch.equal(packed[:, lo:hi], alone)


@pytest.mark.parametrize("shape,h_kv,units", [((2, 1024, 8, 64), 2, 1), ((3, 768, 4, 64), 4, 4),
                                              ((1, 1024, 8, 128), 4, 2),
                                              ((1, 1024, 8, 128), 2, 0.5),   # 2 of 4 heads
                                              ((2, 768, 8, 64), 1, 0.2)])    # 1 of 8 heads
def test_chunked_partials_equal_one_pass(device, monkeypatch, shape, h_kv, units):
    """Per-slot buffers bounded to `units` (batch row, kv head) units: the
    forward and dQ are bitwise the unchunked ones (every stage works per row
    and query head), and so are dK / dV for whole units. Below one unit the
    query heads of a kv head run in subsets whose float32 dK / dV sums are
    added and rounded once, as the one-pass kernel rounds its float32 sum
    once: the two differ only in the order of float32 additions, so by one
    bf16 unit in the last place, plus float32 reassociation error where a
    sum nearly cancels (bounded by 2^-16 of the largest gradient: a few
    hundred float32 terms of at most that size)."""
    from moba.chunking import ENV_BUDGET, unit_bytes

    q, k, v, do = make_qkv(shape, torch.bfloat16, seed=4, n=4)
    k, v = k[:, :, :h_kv].contiguous(), v[:, :, :h_kv].contiguous()
    cfg = MoBAConfig(block_size=128, top_k=4)
    qg, kg, vg, dog = (t.to(device) for t in (q, k, v, do))

    def run():
        fwd = moba_forward(qg, kg, vg, cfg)
        qq, kk, vv = (t.clone().requires_grad_(True) for t in (qg, kg, vg))
        out = moba_attention(qq, kk, vv, cfg)
        out.backward(dog)
        return fwd, out.detach(), qq.grad, kk.grad, vv.grad

    monkeypatch.setenv(ENV_BUDGET, str(1 << 40))
    whole = run()
    unit = unit_bytes(shape[1], shape[2] // h_kv, shape[3], cfg.slots(), 2)
    monkeypatch.setenv(ENV_BUDGET, str(int(units * unit)))
    chunked = run()
    assert torch.equal(whole[0], chunked[0]) and torch.equal(whole[1], chunked[1])
    assert torch.equal(whole[0], whole[1])
    assert torch.equal(whole[2], chunked[2]), "dQ"
    for name, a, b in zip(("dK", "dV"), whole[3:], chunked[3:]):
        if units >= 1:
            assert torch.equal(a, b), name
            continue
        a, b = a.float(), b.float()
        ulp = torch.maximum(a.abs(), b.abs()) * 2.0 ** -7  # >= one bf16 ulp of either
        bound = ulp + a.abs().max() * 2.0 ** -16
        worst = float(((a - b).abs() - bound).max())
        assert worst <= 0, f"{name}: exceeds one ulp + reassociation by {worst}"
        assert max_abs_error(a, b) <= BF16_MAX_ABS and mean_abs_error(a, b) <= BF16_MEAN_ABS, name


def test_chunked_partials_packed(device, monkeypatch):
    """Packed sequences chunk over kv heads; same output as one pass."""
    from moba.chunking import ENV_BUDGET

    lens = [640, 384, 1024]
    cu = torch.tensor([0, 640, 1024, 2048], dtype=torch.int32, device=device)
    q, k, v = (t.to(device) for t in make_qkv((1, sum(lens), 4, 64), torch.bfloat16, seed=6))
    cfg = MoBAConfig(block_size=128, top_k=4)
    monkeypatch.setenv(ENV_BUDGET, str(1 << 40))
    whole = moba_forward(q, k, v, cfg, cu_seqlens=cu, max_seqlen=1024)
    monkeypatch.setenv(ENV_BUDGET, "1")
    chunked = moba_forward(q, k, v, cfg, cu_seqlens=cu, max_seqlen=1024)
    assert torch.equal(whole, chunked)


@pytest.mark.parametrize("shape,h_kv,cu", [((1, 2048, 4, 64), 4, None), ((2, 1024, 8, 128), 2, None),
                                           ((1, 2048, 4, 64), 4, [0, 640, 1024, 2048])])
def test_cut_columns_equal_whole_columns(device, monkeypatch, shape, h_kv, cu):
    """Columns cut into segments (64 entries each, up to 8 per column) give
    the forward and dQ of whole columns bit for bit (every (query, slot)
    result comes from one program either way); dK / dV of cut columns are
    float32 sums of the segments added in order, within the bf16 bars of the
    whole-column result, and repeatable."""
    from moba.kernels.routing import ENV_SEGMENT

    q, k, v, do = make_qkv(shape, torch.bfloat16, seed=9, n=4)
    k, v = k[:, :, :h_kv].contiguous(), v[:, :, :h_kv].contiguous()
    cfg = MoBAConfig(block_size=128, top_k=4)
    qg, kg, vg, dog = (t.to(device) for t in (q, k, v, do))
    cug = None if cu is None else torch.tensor(cu, dtype=torch.int32, device=device)
    mx = None if cu is None else max(b - a for a, b in zip(cu[:-1], cu[1:]))

    def run(index=None):
        if index is None:
            index = build_csc_fused(qg, kg, cfg, cu_seqlens=cug, max_seqlen=mx)
        qq, kk, vv = (t.clone().requires_grad_(True) for t in (qg, kg, vg))
        out = moba_attention(qq, kk, vv, cfg, index=index)
        out.backward(dog)
        return index, out.detach(), qq.grad, kk.grad, vv.grad

    monkeypatch.setenv(ENV_SEGMENT, "0")
    whole = run()
    assert whole[0].segments is None
    monkeypatch.setenv(ENV_SEGMENT, "64")
    cut = run()
    assert int(cut[0].seg_counts[..., 1].sum()) > 0, "no column was cut"
    assert torch.equal(whole[1], cut[1]), "forward changed"
    assert torch.equal(whole[2], cut[2]), "dQ changed"
    for a, b in zip(whole[3:], cut[3:]):
        assert max_abs_error(a.float(), b.float()) <= BF16_MAX_ABS
        assert mean_abs_error(a.float(), b.float()) <= BF16_MEAN_ABS
    again = run(cut[0])  # repeatable given the index (its column order is not fixed)
    assert torch.equal(cut[3], again[3]) and torch.equal(cut[4], again[4])


@pytest.mark.parametrize("dtype,bs,d", [
    (torch.bfloat16, 128, 256), (torch.float16, 64, 256), (torch.float32, 64, 256),
    # a block's keys and values beyond LDS: staged in tiles of keys
    (torch.float32, 128, 256), (torch.bfloat16, 256, 256),
    (torch.bfloat16, 128, 512), (torch.float32, 64, 512),
    (torch.bfloat16, 64, 1024), (torch.float32, 32, 1024)])
def test_large_head_dim_forward_and_backward(device, dtype, bs, d):
    """head_dim 256 to 1024 (the reference's _validate admits any power of
    two, moba_fwd.py:774-776) runs on the FMA kernels, whose key tiles shrink
    with head_dim: forward and gradients against fp64 autograd of the
    oracle, under the dtype's bar."""
    cfg = MoBAConfig(block_size=bs, top_k=4, dtype=dtype)
    shape = (1, 1024, 2, d)
    q, k, v = make_qkv(shape, dtype, seed=31, device=device)
    g = make_qkv(shape, dtype, seed=32, device=device, n=1)[0]
    sel = oracle_selection(q, k, cfg)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = moba_attention(qq, kk, vv, cfg)
    out.backward(g)
    qc, kc, vc, gc = (t.detach().cpu().double().requires_grad_(True) for t in (q, k, v, g))
    ref = O.moba_attention(qc, kc, vc, oracle_cfg(cfg), selected=sel, query_chunk=256)
    ref.backward(gc.detach())
    if dtype == torch.float32:
        for name, ours, tr in (("out", out, ref), ("dq", qq.grad, qc.grad),
                               ("dk", kk.grad, kc.grad), ("dv", vv.grad, vc.grad)):
            assert max_abs_error(ours, tr) <= FP32_MAX_ABS, name
        return
    low = grads_oracle(q, k, v, cfg, sel, g, dtype=dtype)
    lo_out = O.moba_attention(*(t.detach().cpu().to(dtype) for t in (q, k, v)), oracle_cfg(cfg),
                              selected=sel, query_chunk=256)
    for name, ours, tr, lo in (("out", out, ref, lo_out), ("dq", qq.grad, qc.grad, low[0]),
                               ("dk", kk.grad, kc.grad, low[1]), ("dv", vv.grad, vc.grad, low[2])):
        assert_within_tolerance(ours, tr, max_abs_error(lo, tr), name)
        assert mean_abs_error(ours, tr) <= BF16_MEAN_ABS, name


@pytest.mark.parametrize("shape,h_kv,segment", [((1, 1024, 4, 64), 4, "0"),      # MFMA, D 64
                                                ((1, 1024, 8, 128), 2, "0"),     # two streams, D 128
                                                ((1, 2048, 4, 64), 4, "64"),     # cut columns
                                                ((1, 512, 2, 256), 2, "0")])     # FMA fallback
def test_backward_float32_dkdv_rounds_to_the_default(device, monkeypatch, shape, h_kv, segment):
    """moba_backward(dkv_dtype=float32) returns the float32 sums that the
    default call rounds once: rounding them to bf16 gives its dK / dV bit for
    bit, and dQ is unchanged."""
    from moba.kernels.moba_bwd import moba_backward
    from moba.kernels.moba_fwd import attend_partials
    from moba.kernels.routing import ENV_SEGMENT

    monkeypatch.setenv(ENV_SEGMENT, segment)
    cfg = MoBAConfig(block_size=128, top_k=4)
    q, k, v, do = (t.to(device) for t in make_qkv(shape, torch.bfloat16, seed=12, n=4))
    k, v = k[:, :, :h_kv].contiguous(), v[:, :, :h_kv].contiguous()
    index = build_csc_fused(q, k, cfg)
    if segment != "0":
        assert int(index.seg_counts[..., 1].sum()) > 0, "no column was cut"
    part_m, part_l, part_acc = attend_partials(q, k, v, cfg, index)
    out, lse = combine_partials(part_m, part_l, part_acc, q.dtype, return_lse=True)
    dq, dk, dv = moba_backward(do, q, k, v, out, lse, part_m, cfg, index)
    dq32, dk32, dv32 = moba_backward(do, q, k, v, out, lse, part_m, cfg, index,
                                     dkv_dtype=torch.float32)
    assert dk32.dtype is torch.float32 and dv32.dtype is torch.float32
    assert torch.equal(dq, dq32)
    assert torch.equal(dk, dk32.to(torch.bfloat16)) and torch.equal(dv, dv32.to(torch.bfloat16))
    # Not already rounded: some sums carry bits below bf16's precision.
    assert not torch.equal(dk32, dk32.to(torch.bfloat16).float())


def test_packed_gqa_d128_backward_equals_each_sequence_alone(device):
    """The two-stream head_dim-128 backward (128-key blocks) on packed GQA
    input with ragged lengths: columns past a short sequence's end hold no
    keys, and a stream may run a dead step. dQ per query is exact; dK / dV
    sum a column in an order the packing changes, within the bf16 bars."""
    cfg = MoBAConfig(block_size=128, top_k=4)
    lens = [640, 128, 1000, 256]
    cu = torch.tensor([0, 640, 768, 1768, 2024], dtype=torch.int32, device=device)
    t = int(cu[-1])
    q = make_qkv((1, t, 8, 128), torch.bfloat16, seed=15, device=device, n=1)[0]
    k, v = make_qkv((1, t, 2, 128), torch.bfloat16, seed=16, device=device, n=2)
    g = make_qkv((1, t, 8, 128), torch.bfloat16, seed=17, device=device, n=1)[0]
    qq, kk, vv = (x.clone().requires_grad_(True) for x in (q, k, v))
    moba_attention(qq, kk, vv, cfg, cu_seqlens=cu, max_seqlen=max(lens)).backward(g)
    for r, ln in enumerate(lens):
        lo = int(cu[r])
        a = [x[:, lo:lo + ln].clone().requires_grad_(True) for x in (q, k, v)]
        moba_attention(*a, cfg).backward(g[:, lo:lo + ln])
        assert torch.equal(qq.grad[:, lo:lo + ln], a[0].grad), f"dq, sequence {r}"
        for ours, alone in zip((kk.grad, vv.grad), a[1:]):
            assert max_abs_error(ours[:, lo:lo + ln].float(), alone.grad.float()) <= BF16_MAX_ABS, f"sequence {r}"
            assert mean_abs_error(ours[:, lo:lo + ln].float(), alone.grad.float()) <= BF16_MEAN_ABS, f"sequence {r}"
