"""The oracle against the reference oracle's own outputs (tests/golden/).

The fixtures were written by `tests/golden/make_golden.py`, which ran the
reference's `pool_blocks_naive`, `gate_select_naive`, `moba_selection` and
`moba_attention_naive` on seeded inputs. Inputs are regenerated here from the
same seeds and checked against the stored digests first, so a drift in the
generator cannot masquerade as an oracle bug.
"""

import hashlib
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import oracle_cfg
from oracle import c_oracle
from oracle import naive as O

GOLDEN = np.load(Path(__file__).resolve().parent / "golden" / "reference_oracle.npz")
DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def cfg(bs, tk, **kw):
    from moba.config import MoBAConfig
    return oracle_cfg(MoBAConfig(block_size=bs, top_k=tk, **kw))


def ref_qkv(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(shape, generator=g, dtype=dtype) for _ in range(3))


def digest(*ts):
    h = hashlib.sha256()
    for t in ts:
        h.update(t.contiguous().view(torch.uint8).numpy().tobytes())
    return h.hexdigest()


GATE_CASES = sorted(k[:-6] for k in GOLDEN.files if k.endswith("__meta"))


def gate_inputs(name):
    b, s, h, d, bs, tk, seed, hkv, dtc = (int(x) for x in GOLDEN[name + "__meta"])
    q, k, _ = ref_qkv((b, s, h, d), DTYPES[dtc], seed)
    k = k[:, :, :hkv].contiguous()
    assert digest(q, k) == str(GOLDEN[name + "__digest"]), "input generator drifted"
    return q, k, bs, tk


@pytest.mark.parametrize("name", GATE_CASES)
def test_pool_matches_reference_bitwise(name):
    q, k, bs, tk = gate_inputs(name)
    kbar = O.pool_blocks(k, bs)
    assert np.array_equal(kbar.view(torch.int16).numpy(), GOLDEN[name + "__kbar_bits"])


@pytest.mark.parametrize("name", GATE_CASES)
def test_selection_matches_reference_exactly(name):
    q, k, bs, tk = gate_inputs(name)
    c = cfg(bs, tk)
    sel = O.gate_select(q, O.pool_blocks(k, bs), c)
    idx = O.mask_to_indices(sel, tk).numpy()
    assert np.array_equal(idx, GOLDEN[name + "__idx"])


@pytest.mark.parametrize("name", GATE_CASES)
def test_selection_logic_matches_reference_on_its_own_scores(name):
    """Fed the reference's float32-einsum scores, the oracle's selection rule
    (mask, stable sort, budget, -inf drop, own block) reproduces the
    reference bit for bit -- this pins the rule independently of rounding."""
    q, k, bs, tk = gate_inputs(name)
    kbar = O.pool_blocks(k, bs)
    scores = torch.einsum("bshd,bhnd->bhsn", q, O.expand_kv(kbar, q.shape[2], dim=1))
    idx = O.mask_to_indices(O.select_from_scores(scores, cfg(bs, tk)), tk).numpy()
    assert np.array_equal(idx, GOLDEN[name + "__idx"])


@pytest.mark.parametrize("name", GATE_CASES)
def test_c_oracle_matches_reference(name):
    q, k, bs, tk = gate_inputs(name)
    kbar = c_oracle.pool_blocks(k, bs)
    assert np.array_equal(kbar.view(torch.int16).numpy(), GOLDEN[name + "__kbar_bits"])
    idx = c_oracle.gate_select(q, kbar, cfg(bs, tk)).numpy()
    assert np.array_equal(idx, GOLDEN[name + "__idx"])


def test_forced_ties_resolve_like_reference():
    q, k, _ = ref_qkv((1, 512, 1, 64), torch.bfloat16, 0)
    assert digest(q, k) == str(GOLDEN["ties__digest"])
    kbar = torch.from_numpy(GOLDEN["ties__kbar_bits"]).view(torch.bfloat16)
    c = cfg(64, 2)
    assert np.array_equal(O.mask_to_indices(O.gate_select(q, kbar, c), 2).numpy(),
                          GOLDEN["ties__idx"])
    assert np.array_equal(c_oracle.gate_select(q, kbar, c).numpy(), GOLDEN["ties__idx"])


def test_varlen_selection_matches_reference():
    cu = torch.from_numpy(GOLDEN["varlen__cu"])
    q, k, _ = ref_qkv((1, 212, 2, 64), torch.bfloat16, 5)
    assert digest(q, k) == str(GOLDEN["varlen__digest"])
    c = cfg(16, 3)
    sel = O.moba_selection(q, k, c, cu_seqlens=cu)
    assert np.array_equal(O.mask_to_indices(sel, 3).numpy(), GOLDEN["varlen__idx"])
    kb = c_oracle.pool_blocks(k, 16, cu, 80)
    assert np.array_equal(c_oracle.gate_select(q, kb, c, cu, 80).numpy(),
                          GOLDEN["varlen__idx"])


@pytest.mark.parametrize("tag,kw", [("nocur", dict(always_select_current=False)),
                                    ("excl", dict(top_k_includes_current=False))])
def test_nondefault_flags_match_reference(tag, kw):
    q, k, _ = ref_qkv((1, 512, 2, 64), torch.bfloat16, 6)
    assert digest(q, k) == str(GOLDEN[f"{tag}__digest"])
    c = cfg(32, 3, **kw)
    sel = O.moba_selection(q, k, c)
    assert np.array_equal(O.mask_to_indices(sel, 4).numpy(), GOLDEN[f"{tag}__idx"])


def test_config1_fp32_attention_matches_reference():
    """fp32 [1,4096,4,64], bs128 k8 on the CPU oracle."""
    q, k, v = ref_qkv((1, 4096, 4, 64), torch.float32, 0)
    assert digest(q, k, v) == str(GOLDEN["cfg1__digest"])
    c = cfg(128, 8)
    sel = O.moba_selection(q, k, c)
    assert np.array_equal(O.mask_to_indices(sel, 8).numpy(), GOLDEN["cfg1__idx"])
    rows = torch.from_numpy(GOLDEN["cfg1__rows"])
    o = O.moba_attention(q, k, v, c, selected=sel, query_chunk=512)
    np.testing.assert_allclose(o[:, rows].numpy(), GOLDEN["cfg1__out_rows"],
                               atol=2e-6, rtol=0)
    s1, s2 = GOLDEN["cfg1__out_sum"]
    assert abs(o.double().sum().item() - s1) < 1e-2
    assert abs(o.double().square().sum().item() - s2) < 1e-2


@pytest.mark.parametrize("name,shape,h_kv,bs,tk,seed",
                         [("a64_gqa", (1, 256, 4, 32), 2, 32, 3, 7),
                          ("a64_tail", (1, 200, 2, 32), 2, 64, 2, 8)])
def test_fp64_attention_matches_reference(name, shape, h_kv, bs, tk, seed):
    q, k, v = ref_qkv(shape, torch.float64, seed)
    k, v = k[:, :, :h_kv].contiguous(), v[:, :, :h_kv].contiguous()
    assert digest(q, k, v) == str(GOLDEN[name + "__digest"])
    o = O.moba_attention(q, k, v, cfg(bs, tk))
    np.testing.assert_allclose(o.numpy(), GOLDEN[name + "__out"], atol=1e-12, rtol=0)


def test_fp64_packed_attention_matches_reference():
    cu = torch.from_numpy(GOLDEN["varlen__cu"])
    q, k, v = ref_qkv((1, 212, 2, 32), torch.float64, 9)
    assert digest(q, k, v) == str(GOLDEN["avarlen__digest"])
    o = O.moba_attention(q, k, v, cfg(16, 3), cu_seqlens=cu)
    np.testing.assert_allclose(o.numpy(), GOLDEN["avarlen__out"], atol=1e-12, rtol=0)
