"""Pool and gate on the GPU against the oracle: bitwise kbar, exact ids."""

import pytest
import torch

from conftest import GATE_SWEEP, SHAPE_SWEEP, make_qkv, oracle_cfg, sweep_cases
from moba.config import MoBAConfig
from moba.kernels.gating import gate_select
from moba.kernels.pooling import pool_blocks
from oracle import c_oracle
from oracle import naive as O

pytestmark = pytest.mark.gpu


def run_gate(q, k, cfg, cu=None, mx=None):
    kbar = pool_blocks(k, cfg, cu_seqlens=cu, max_seqlen=mx)
    return kbar, gate_select(q, kbar, cfg, cu_seqlens=cu, max_seqlen=mx)


def check(q, k, cfg, cu=None, mx=None):
    kbar, idx = run_gate(q, k, cfg, cu, mx)
    kc = k.cpu()
    cuc = None if cu is None else cu.cpu()
    ref_kbar = c_oracle.pool_blocks(kc, cfg.block_size, cuc, mx)
    got_kbar = kbar.cpu()
    if cu is not None:  # only rows a sequence owns are defined
        lens = (cuc[1:] - cuc[:-1]).tolist()
        for r, ln in enumerate(lens):
            nb = -(-ln // cfg.block_size)
            assert torch.equal(got_kbar[r, :, :nb], ref_kbar[r, :, :nb]), f"kbar row {r}"
    else:
        assert torch.equal(got_kbar, ref_kbar), "kbar differs from the oracle"
    ref = c_oracle.gate_select(q.cpu(), ref_kbar, oracle_cfg(cfg), cuc, mx)
    got = idx.cpu()
    bad = (got != ref).any(-1)
    assert not bool(bad.any()), (
        f"{int(bad.sum())} queries route differently; first {torch.nonzero(bad)[0].tolist()}: "
        f"got {got[bad][0].tolist()} want {ref[bad][0].tolist()}")
    return idx


@pytest.mark.parametrize("shape,gate", sweep_cases())
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gate_matches_oracle(device, shape, gate, dtype):
    cfg = MoBAConfig(block_size=gate[0], top_k=gate[1], dtype=dtype)
    q, k, _ = make_qkv(shape, dtype, device=device)
    check(q, k, cfg)


@pytest.mark.parametrize("gate", [(128, 8), (64, 4)])
def test_gate_fp32(device, gate):
    cfg = MoBAConfig(block_size=gate[0], top_k=gate[1], dtype=torch.float32)
    q, k, _ = make_qkv((1, 2048, 2, 64), torch.float32, device=device)
    check(q, k, cfg)


def test_gate_forced_ties_go_to_block_zero(device):
    cfg = MoBAConfig(block_size=64, top_k=2)
    q, k, _ = make_qkv((1, 512, 1, 64), torch.bfloat16, device=device)
    kbar = pool_blocks(k, cfg)
    kbar[:] = kbar[:, :, :1, :]
    idx = gate_select(q, kbar, cfg)
    assert int(idx[0, 0, 400, 0]) == 0
    ref = c_oracle.gate_select(q.cpu(), kbar.cpu(), oracle_cfg(cfg))
    assert torch.equal(idx.cpu(), ref)
    assert torch.equal(idx, gate_select(q, kbar, cfg)), "gate is not repeatable"


@pytest.mark.parametrize("shape,bs,tk", [((1, 512, 2, 64), 128, 12),    # budget > blocks
                                         ((1, 16384, 1, 64), 32, 64),   # 512 blocks, k=64
                                         ((1, 1000, 2, 128), 128, 8),   # ragged tail
                                         ((1, 3000, 2, 64), 96, 5),     # non-pow2 block
                                         ((1, 2048, 2, 64), 128, 1)])   # own block only
def test_gate_edge_shapes(device, shape, bs, tk):
    cfg = MoBAConfig(block_size=bs, top_k=tk)
    q, k, _ = make_qkv(shape, torch.bfloat16, seed=2, device=device)
    check(q, k, cfg)


@pytest.mark.parametrize("hq,hkv,d", [(8, 2, 128), (32, 8, 128), (4, 1, 64)])
def test_gate_gqa_ranks_per_query_head(device, hq, hkv, d):
    cfg = MoBAConfig(block_size=64, top_k=4)
    q, k, _ = make_qkv((1, 2048, hq, d), torch.bfloat16, seed=3, device=device)
    k = k[:, :, :hkv].contiguous()
    idx = check(q, k, cfg)
    # heads sharing a kv head still choose differently
    assert not torch.equal(idx[0, 0], idx[0, 1])


@pytest.mark.parametrize("lens,bs,tk", [([80, 48, 64, 20], 16, 3),
                                        ([2048, 130, 4000, 777], 128, 8)])
def test_gate_packed(device, lens, bs, tk):
    cfg = MoBAConfig(block_size=bs, top_k=tk)
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    q, k, _ = make_qkv((1, int(cu[-1]), 2, 64), torch.bfloat16, seed=5, device=device)
    idx = check(q, k, cfg, cu.to(device), max(lens))
    # no selected block crosses a sequence boundary (ids are sequence-local)
    for r, ln in enumerate(lens):
        lo = int(cu[r])
        blk = idx[0, :, lo:lo + ln]
        assert int(blk.max()) < -(-ln // bs)


@pytest.mark.parametrize("flags", [dict(always_select_current=False),
                                   dict(top_k_includes_current=False)])
def test_gate_nondefault_flags(device, flags):
    cfg = MoBAConfig(block_size=32, top_k=3, **flags)
    q, k, _ = make_qkv((1, 1024, 2, 64), torch.bfloat16, seed=6, device=device)
    check(q, k, cfg)


def test_gate_full_size_config2(device):
    """BASELINE config 2 routing: [1, 65536, 4, 64] bf16, bs128, k8."""
    cfg = MoBAConfig(block_size=128, top_k=8)
    q, k, _ = make_qkv((1, 65536, 4, 64), torch.bfloat16, seed=0, device=device)
    check(q, k, cfg)


@pytest.mark.parametrize("d,bs,tk", [(64, 128, 8), (128, 64, 8), (64, 32, 13)])
def test_gate_integer_inputs_with_many_exact_ties(device, d, bs, tk):
    """Small-integer q and k make equal scores common: the lowest-index
    tie-break and the approximate-then-exact retention must still agree with
    the oracle bit for bit (many queries take the exact fallback here)."""
    cfg = MoBAConfig(block_size=bs, top_k=tk)
    g = torch.Generator().manual_seed(21)
    q = torch.randint(-2, 3, (1, 8192, 2, d), generator=g).to(torch.bfloat16).to(device)
    k = torch.randint(-1, 2, (1, 8192, 2, d), generator=g).to(torch.bfloat16).to(device)
    check(q, k, cfg)


@pytest.mark.parametrize("d", [64, 128])
def test_gate_every_score_a_candidate(device, d):
    """Scores rising block by block ((j + 1) / 64 per feature of block j,
    all-ones queries): with two 32-block chunks pass 1 finds fewer than
    `take` chunk maxima, so the threshold stays at -inf, every score of pass
    2 is a candidate and every group appends all four scores; the per-lane
    buffer must be folded often enough that no candidate is lost."""
    cfg = MoBAConfig(block_size=128, top_k=8)
    S = 8192
    j = torch.arange(S) // 128
    k = ((j + 1).float() / 64).view(1, S, 1, 1).expand(1, S, 1, d) / (d // 8)
    k = k.to(torch.bfloat16).contiguous().to(device)
    q = torch.ones(1, S, 1, d, dtype=torch.bfloat16, device=device)
    idx = check(q, k, cfg)
    last = idx[0, 0, -1].tolist()  # the last query: own block 63, top 7 of 0..62
    assert last == list(range(56, 64)), last


@pytest.mark.parametrize("d", [64, 128])
def test_gate_overflowing_scores_tie_to_the_lowest_blocks(device, d):
    """q and k near 1e19: every dot product exceeds float32's range, so every
    score is +inf and every strictly-past block ties. The gate cannot bound
    such scores and sends the queries to its exact queue kernel, whose
    selection must be the oracle's: the lowest block ids."""
    cfg = MoBAConfig(block_size=128, top_k=8)
    S = 2048
    q = torch.full((1, S, 2, d), 1e19, dtype=torch.bfloat16, device=device)
    k = torch.full((1, S, 2, d), 1e19, dtype=torch.bfloat16, device=device)
    idx = check(q, k, cfg)
    last = idx[0, 0, -1].tolist()  # own block 15, the 7 lowest past blocks
    assert last == [0, 1, 2, 3, 4, 5, 6, 15], last


def _structured_keys(kind, shape, dtype, seed, device):
    """Keys whose block representatives nearly coincide, so that many scores
    round to equal values of the storage dtype: a shared per-channel offset
    plus noise ("bias", as trained keys carry), or a slow random walk over
    the tokens ("walk")."""
    g = torch.Generator().manual_seed(seed)
    if kind == "bias":
        k = 3.0 * torch.randn((1, 1) + tuple(shape[2:]), generator=g) + torch.randn(shape, generator=g)
    else:
        k = (torch.randn(shape, generator=g) * 0.05).cumsum(1)
    return k.to(dtype).to(device)


@pytest.mark.parametrize("kind", ["bias", "walk"])
@pytest.mark.parametrize("d,gate", [(64, (64, 8)), (128, (64, 8)), (64, (32, 17)), (128, (128, 12))])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gate_near_tied_keys_match_oracle(device, kind, d, gate, dtype):
    """Many candidates share a rounded score: the order among them is the
    block id, which the gate must reproduce exactly."""
    cfg = MoBAConfig(block_size=gate[0], top_k=gate[1], dtype=dtype)
    shape = (1, 8192, 2, d)
    q = make_qkv(shape, dtype, seed=31, device=device, n=1)[0]
    k = _structured_keys(kind, shape, dtype, 32, device)
    check(q, k, cfg)


@pytest.mark.parametrize("dtype,scale", [
    (torch.bfloat16, 1e-19), (torch.bfloat16, 1e-12), (torch.bfloat16, 1e12),
    (torch.float16, 0.02), (torch.float16, 20.0),
])
def test_gate_near_tied_keys_at_extreme_scales(device, dtype, scale):
    """Offset keys scaled so that the scores sit among subnormal or very large
    rounded values (the key intervals and the threshold below the bound then
    meet the format's edges), and, for float16, near its overflow."""
    cfg = MoBAConfig(block_size=64, top_k=8, dtype=dtype)
    shape = (1, 4096, 2, 64)
    q = (make_qkv(shape, torch.float32, seed=35, device=device, n=1)[0] * scale).to(dtype)
    k = (_structured_keys("bias", shape, torch.float32, 36, device) * scale).to(dtype)
    check(q, k, cfg)


@pytest.mark.parametrize("kind", ["bias", "walk"])
def test_gate_near_tied_keys_packed_gqa_match_oracle(device, kind):
    """Near-tied keys through the packed path with grouped query heads."""
    cfg = MoBAConfig(block_size=64, top_k=8, dtype=torch.bfloat16)
    lens = [3000, 517, 4096, 1200]
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    t = int(cu[-1])
    q = make_qkv((1, t, 4, 64), torch.bfloat16, seed=37, device=device, n=1)[0]
    k = _structured_keys(kind, (1, t, 2, 64), torch.bfloat16, 38, device)
    check(q, k, cfg, cu.to(device), max(lens))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gate_fallback_settles_heavy_ties_exactly(device, dtype):
    """Keys dominated by one shared offset: scores spread over only a few
    rounded values, so the boundary key is shared by more candidates than
    the first kernel's lists hold. Those queries must reach the fallback
    kernel (its tile counter, the second word of the workspace, is
    non-zero), whose lists rank by (key, id) and so settle the ties by id,
    and come out as the oracle selects them. Queries the fallback cannot
    settle either go on to the exact queue (the first word)."""
    from moba import _lib

    cfg = MoBAConfig(block_size=64, top_k=8, dtype=dtype)
    shape = (1, 8192, 2, 64)
    g = torch.Generator().manual_seed(39)
    # float16 keys are finer (10 mantissa bits), so its offset is larger:
    # scores near 800, where a float16 step (0.5) is twice their spread.
    scale, offset = (1.0, 8.0) if dtype is torch.bfloat16 else (0.5, 48.0)
    q = (torch.randn(shape, generator=g) * scale).to(dtype).to(device)
    k = ((offset * torch.randn((1, 1, 2, 64), generator=g) + torch.randn(shape, generator=g))
         * scale).to(dtype).to(device)
    kbar = pool_blocks(k, cfg)
    b, s, h, d = q.shape
    n = kbar.shape[2]
    ws = torch.zeros(int(_lib.load().moba_gate_workspace_size(b, s, h)), dtype=torch.uint8,
                     device=device)
    out = torch.empty((b, h, s, cfg.slots()), dtype=torch.int32, device=device)
    _lib.call("moba_gate", _lib.ptr(q), _lib.ptr(kbar), _lib.ptr(out), None, b, s, s, h, h, d, n,
              cfg.block_size, cfg.slots(), cfg.past_blocks_selected(n), 1,
              _lib.DTYPE_CODE[dtype], _lib.ptr(ws), ws.numel(), _lib.stream_handle(device))
    queued, fallback = ws[:8].view(torch.int32).tolist()
    print(f"[heavy ties] {dtype}: fallback tiles {fallback}, queued {queued}", flush=True)
    assert fallback > 0, "no query reached the fallback kernel"
    ref = c_oracle.gate_select(q.cpu(), kbar.cpu(), oracle_cfg(cfg))
    bad = (out.cpu() != ref).any(-1)
    assert not bool(bad.any()), f"{int(bad.sum())} queries differ"


def _gate_with_counters(q, kbar, cfg, cu=None, mx=None):
    """moba_gate with its own workspace: the ids and the workspace's two
    counters (queries sent to the exact queue, tiles the fallback kernel
    ran)."""
    from moba import _lib

    b, s, h, d = q.shape
    rows = s if cu is None else mx          # rows per sequence
    seqs = b if cu is None else cu.numel() - 1  # the C call's batch: sequences when packed
    n = kbar.shape[2]
    ws = torch.zeros(int(_lib.load().moba_gate_workspace_size(seqs, rows, h)),
                     dtype=torch.uint8, device=q.device)
    out = torch.full((b, h, s, cfg.slots()), -7, dtype=torch.int32, device=q.device)
    take = cfg.past_blocks_selected(-(-rows // cfg.block_size))
    _lib.call("moba_gate", _lib.ptr(q), _lib.ptr(kbar), _lib.ptr(out),
              None if cu is None else _lib.ptr(cu), seqs, s, rows, h, kbar.shape[1], d, n,
              cfg.block_size, cfg.slots(), take, int(bool(cfg.always_select_current)),
              _lib.DTYPE_CODE[q.dtype], _lib.ptr(ws), ws.numel(), _lib.stream_handle(q.device))
    torch.cuda.synchronize()
    queued, tiles = ws[:8].view(torch.int32).tolist()
    return out, queued, tiles


def _heavy_tie_keys(shape, dtype, seed, device):
    """One shared per-channel offset, 8 times the noise: scores take only a
    few rounded values, so many queries of a workgroup stay unsettled."""
    g = torch.Generator().manual_seed(seed)
    k = 8.0 * torch.randn((1, 1) + tuple(shape[2:]), generator=g) + torch.randn(shape, generator=g)
    return k.to(dtype).to(device)


@pytest.mark.parametrize("case", ["packed_gqa", "d128", "take16_bs32", "multi_tile_lists",
                                  "append_wide_ids"])
def test_gate_fallback_kernel_paths_match_oracle(device, case):
    """Shared-offset keys leave many queries of a workgroup unsettled, so the
    first kernel hands them to the fallback kernel (its tile counter is
    non-zero): through packed sequences with grouped query heads, at head
    dim 128, at take 16 with 32-key blocks, with lists long enough that
    several tiles of one list are spread over the workgroups striding over
    it, and with more groups than a float16 key's 13 free low bits can name
    next to a slot (8192 blocks at take 16), where the fallback kernel
    appends scores to lists instead of tracking keyed groups. Every id as
    the oracle selects it (every fourth query in the last case)."""
    dtype = torch.bfloat16
    cu = mx = None
    if case == "packed_gqa":
        cfg = MoBAConfig(block_size=64, top_k=8, dtype=dtype)
        lens = [8192, 517, 6000, 1200]
        cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32,
                          device=device)
        mx = max(lens)
        t = int(cu[-1])
        q = make_qkv((1, t, 4, 64), dtype, seed=41, device=device, n=1)[0]
        k = _heavy_tie_keys((1, t, 2, 64), dtype, 42, device)
    elif case == "d128":
        cfg = MoBAConfig(block_size=64, top_k=8, dtype=dtype)
        q = make_qkv((1, 8192, 2, 128), dtype, seed=43, device=device, n=1)[0]
        k = _heavy_tie_keys((1, 8192, 2, 128), dtype, 44, device)
    elif case == "take16_bs32":
        cfg = MoBAConfig(block_size=32, top_k=17, dtype=dtype)
        q = make_qkv((1, 8192, 2, 64), dtype, seed=45, device=device, n=1)[0]
        k = _heavy_tie_keys((1, 8192, 2, 64), dtype, 46, device)
    elif case == "multi_tile_lists":
        cfg = MoBAConfig(block_size=64, top_k=8, dtype=dtype)
        q = make_qkv((1, 65536, 2, 64), dtype, seed=47, device=device, n=1)[0]
        k = _heavy_tie_keys((1, 65536, 2, 64), dtype, 48, device)
    else:
        dtype = torch.float16
        cfg = MoBAConfig(block_size=16, top_k=17, dtype=dtype)
        q = make_qkv((1, 131072, 2, 64), dtype, seed=49, device=device, n=1)[0]
        k = _heavy_tie_keys((1, 131072, 2, 64), dtype, 50, device)
    kbar = pool_blocks(k, cfg, cu_seqlens=cu, max_seqlen=mx)
    got, queued, tiles = _gate_with_counters(q, kbar, cfg, cu, mx)
    print(f"[fallback paths] {case}: fallback tiles {tiles}, queued {queued}", flush=True)
    if case == "append_wide_ids":
        ref = c_oracle.gate_select_strided(q.cpu(), kbar.cpu(), oracle_cfg(cfg), stride=4)
        got = got[:, :, ::4]
    else:
        ref = c_oracle.gate_select(q.cpu(), kbar.cpu(), oracle_cfg(cfg),
                                   None if cu is None else cu.cpu(), mx)
    bad = (got.cpu() != ref).any(-1)
    assert not bool(bad.any()), (
        f"{int(bad.sum())} queries route differently; first {torch.nonzero(bad)[0].tolist()}")
    assert tiles > 0, "no query reached the fallback kernel"
    if case == "multi_tile_lists":
        # 2 heads x 16 buckets: more tiles than lists means lists of several tiles
        assert tiles > 2 * 16, tiles
