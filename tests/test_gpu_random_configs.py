"""Randomly drawn configurations, fixed seeds: batch, length (not a multiple of
the block size), query / kv heads, head_dim, block size, top_k, dtype and
packed sequences vary together, so combinations the fixed sweeps do not
list are covered. Per case: the CSC index's selection equals the oracle's
exactly (`naive.py:64-146` via `oracle.naive.moba_selection`); output and
dQ / dK / dV are within the relative tolerance policy of `tolerance.py`
against the fp64 oracle with the selection held fixed.
"""

import random

import pytest
import torch

from conftest import oracle_cfg
from gpu_util import fp64_truth, oracle_selection
from moba.config import MoBAConfig
from moba.kernels.attention import moba_attention
from moba.kernels.routing import build_csc_fused, csc_to_mask
from oracle import naive as O
from tolerance import assert_selection_matches, assert_within_tolerance, max_abs_error

pytestmark = pytest.mark.gpu


def draw(seed):
    """One configuration from a seed: (cfg, b, s, hq, h_kv, d, lens or None)."""
    r = random.Random(seed)
    bs = r.choice([32, 64, 128])
    d = r.choice([64, 64, 128])
    h_kv = r.choice([1, 2, 4])
    hq = h_kv * r.choice([1, 1, 2, 4])
    dtype = r.choice([torch.bfloat16, torch.bfloat16, torch.float16, torch.float32])
    lens = None
    if r.random() < 0.3:
        lens = [r.randint(1, 12) * bs + r.choice([0, r.randint(1, bs - 1)])
                for _ in range(r.randint(2, 4))]
        b, s, nb = 1, sum(lens), -(-max(lens) // bs)
    else:
        b = r.choice([1, 2])
        s = r.randint(4, 24) * bs + r.choice([0, r.randint(1, bs - 1)])
        nb = -(-s // bs)
    top_k = r.randint(1, min(12, nb))
    return MoBAConfig(block_size=bs, top_k=top_k, dtype=dtype), b, s, hq, h_kv, d, lens


@pytest.mark.parametrize("seed", range(12))
def test_random_configuration_matches_oracle(device, seed):
    cfg, b, s, hq, h_kv, d, lens = draw(1000 + seed)
    print(f"[random-config {seed}] b{b} s{s} hq{hq} hkv{h_kv} d{d} bs{cfg.block_size} "
          f"k{cfg.top_k} {cfg.dtype} lens={lens}", flush=True)
    g = torch.Generator().manual_seed(seed)
    q, k, v, do = (torch.randn((b, s, h, d), generator=g).to(cfg.dtype)
                   for h in (hq, h_kv, h_kv, hq))
    cu = None if lens is None else torch.tensor([0] + lens).cumsum(0).to(torch.int32)
    kw = {} if cu is None else {"cu_seqlens": cu.to(device), "max_seqlen": max(lens)}
    qd, kd, vd, dod = (t.to(device) for t in (q, k, v, do))

    sel = oracle_selection(q, k, cfg, cu_seqlens=cu)
    assert_selection_matches(csc_to_mask(build_csc_fused(qd, kd, cfg, **kw), s), sel, "index")

    qq, kk, vv = (t.clone().requires_grad_(True) for t in (qd, kd, vd))
    out = moba_attention(qq, kk, vv, cfg, **kw)
    out.backward(dod)
    truth, ref_err = fp64_truth(q, k, v, cfg, sel, cu_seqlens=cu)
    assert_within_tolerance(out, truth, ref_err, "out")

    def grads(dtype):
        qc, kc, vc = (t.to(dtype).requires_grad_(True) for t in (q, k, v))
        O.moba_attention(qc, kc, vc, oracle_cfg(cfg), selected=sel, query_chunk=256,
                         cu_seqlens=cu).backward(do.to(dtype))
        return qc.grad, kc.grad, vc.grad

    truth_g, low_g = grads(torch.float64), grads(cfg.dtype)
    for name, ours, t, low in zip(("dq", "dk", "dv"), (qq.grad, kk.grad, vv.grad),
                                  truth_g, low_g):
        assert_within_tolerance(ours, t, max_abs_error(low, t), name)
