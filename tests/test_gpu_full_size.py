"""Parity at BASELINE.json's full sizes, where the dense oracle cannot run.

Cases: config 2 (fwd, [1,65536,4,64]), config 3 (fwd+bwd, [1,131072,4,64]),
config 4 (GQA fwd+bwd, S=32768, Hq=32, Hkv=8, D=128), config 5 (varlen
fwd+bwd, 8 sequences of U[2048,131072] tokens rounded to 128, ~512K packed)
and the headline fwd+bwd [1,524288,4,64]; all bf16, block_size 128, top_k 8,
causal, inputs i.i.d. N(0,1) from a seeded CPU generator.

What is checked, per sequence:
* pool: the whole kbar, bitwise, against the C oracle;
* gate: the selected ids of sampled query rows, exactly, against the oracle
  restricted to those rows (`oracle.naive.gate_select_rows`);
* O and dQ of sampled query rows against the float64 sparse-gather oracle
  with the routing held fixed (a query's output and dQ depend only on its
  own row, its selected blocks and dO);
* dK and dV of sampled KV blocks against the same oracle run over every
  query that selected one of those blocks (all of a key's gradient comes
  from those queries).
* dK and dV of the earliest blocks (0 and 1), the longest columns: every
  query of a sequence may pick block 0, so its column holds ~7 bs ln(nb)
  entries per head, the column the segment list cuts and the longest
  reductions of the backward. Checked for one kv head (its whole query-head
  group) to bound the oracle's cost.
Tolerances (bf16):
* O: the north star's bars, max-abs <= 2e-2 and mean-abs <= 2e-3;
* dQ, dK, dV: the reference's policy (tests/tolerance.py:145-170), max-abs
  error against the float64 oracle within 2x that of the same oracle run in
  bfloat16 on the same rows and keys; and, as well, the north star's bars
  made scale-aware for gradients that sum over many queries: max-abs <=
  2e-2 * max(1, max|truth|), mean-abs <= 2e-3 * max(1, mean|truth|).
"""

import pytest
import torch

from conftest import make_qkv, oracle_cfg
from oracle import c_oracle as C
from oracle import naive as O
from tolerance import assert_selection_matches, assert_within_tolerance, max_abs_error

pytestmark = pytest.mark.gpu

BS, TOPK = 128, 8
MAX_GATHER_BYTES = 1 << 30  # float64 gather budget of one oracle chunk


def _cfg():
    from moba.config import MoBAConfig
    return MoBAConfig(block_size=BS, top_k=TOPK)


def _abs_bars(actual, truth, name):
    err = (actual.double() - truth.double()).abs()
    assert err.max().item() <= 2e-2, f"{name}: max-abs {err.max().item():.3e} > 2e-2"
    assert err.mean().item() <= 2e-3, f"{name}: mean-abs {err.mean().item():.3e} > 2e-3"


def _grad_bars(actual, truth, low, name):
    """The reference's 2x-same-dtype-oracle policy, then the scale-aware bars."""
    assert_within_tolerance(actual, truth, max_abs_error(low, truth), name)
    _bars(actual, truth, name)


def _bars(actual, truth, name):
    a, t = actual.double(), truth.double()
    err = (a - t).abs()
    mx, mean = err.max().item(), err.mean().item()
    lim_mx = 2e-2 * max(1.0, t.abs().max().item())
    lim_mean = 2e-3 * max(1.0, t.abs().mean().item())
    assert mx <= lim_mx, f"{name}: max-abs {mx:.3e} > {lim_mx:.3e}"
    assert mean <= lim_mean, f"{name}: mean-abs {mean:.3e} > {lim_mean:.3e}"


def _sample_rows(length, n=48):
    rows = {0, 1, BS - 1, BS, length // 2, length - BS, length - 2, length - 1}
    step = max(1, length // n)
    rows.update(range(3, length, step))
    return torch.tensor(sorted(r for r in rows if 0 <= r < length))


def _oracle(q, k, v, do, idx, rows, key_blocks=None, dtype=torch.float64, key_users_only=False):
    """`oracle.naive.sparse_grads` on CPU tensors: (out, dq) of `rows` and
    dK / dV of the keys of `key_blocks` from those rows."""
    return O.sparse_grads(q, k, v, do, idx, BS, rows, key_blocks=key_blocks, dtype=dtype,
                          max_gather_bytes=MAX_GATHER_BYTES, key_users_only=key_users_only)


def _check_blocks(name, q, k, v, do, idx, dk, dv, blocks, kv_head=None):
    """dK / dV of `blocks` against the float64 and bfloat16 oracles run over
    every query that selected one of them: of every kv head, or of the
    query-head group of `kv_head` alone."""
    h_q, h_kv = q.shape[2], k.shape[2]
    if kv_head is not None:
        g = h_q // h_kv
        hs = slice(kv_head * g, (kv_head + 1) * g)
        q, do, idx = q[:, :, hs], do[:, :, hs], idx[:, hs]
        k, v = k[:, :, kv_head:kv_head + 1], v[:, :, kv_head:kv_head + 1]
        dk, dv = dk[:, :, kv_head:kv_head + 1], dv[:, :, kv_head:kv_head + 1]
        name = f"{name} kv head {kv_head}"
    length = q.shape[1]
    hit = (idx[..., None] == torch.tensor(blocks)).any(-1).any(-1).any(1)[0]   # [L]
    users = torch.nonzero(hit).flatten()
    keys = torch.cat([torch.arange(b * BS, min((b + 1) * BS, length)) for b in blocks])
    truth = _oracle(q, k, v, do, idx, users, blocks, key_users_only=True)
    low = _oracle(q, k, v, do, idx, users, blocks, dtype=torch.bfloat16, key_users_only=True)
    label = f"{name} blocks {blocks} ({users.numel()} queries)"
    _grad_bars(dk[:, keys], truth[2][:, keys], low[2][:, keys], f"{label} dK")
    _grad_bars(dv[:, keys], truth[3][:, keys], low[3][:, keys], f"{label} dV")


def _check_sequence(name, q, k, v, do, kbar, idx, out, dq, dk, dv, bwd, blocks,
                    early_kv_head=0):
    """All tensors CPU, one sequence: q/k/v/do/out/dq/dk/dv `[1, L, H, D]`,
    kbar `[1, Hkv, nb, D]` (GPU result), idx `[1, Hq, L, slots]` (GPU)."""
    cfg = _cfg()
    length = q.shape[1]
    rows = _sample_rows(length)
    # gate, exactly, on the sampled rows
    want = O.mask_to_indices(O.gate_select_rows(q, kbar, oracle_cfg(cfg), rows),
                             idx.shape[-1])
    assert_selection_matches(idx[:, :, rows], want, f"{name} gate rows")
    # O and dQ of the sampled rows
    truth = _oracle(q, k, v, do, idx, rows, key_blocks=[])
    _abs_bars(out[:, rows], truth[0], f"{name} O rows")
    if not bwd:
        return
    low = _oracle(q, k, v, do, idx, rows, key_blocks=[], dtype=torch.bfloat16)
    _grad_bars(dq[:, rows], truth[1], low[1], f"{name} dQ rows")
    # dK / dV of sampled late blocks, from every query that selected them
    _check_blocks(name, q, k, v, do, idx, dk, dv, blocks)
    # ... and of the two earliest, longest columns, for one kv head
    _check_blocks(name, q, k, v, do, idx, dk, dv, [0, 1], kv_head=early_kv_head)


def _run(shape, h_kv, bwd, lens=None):
    from moba.kernels.attention import moba_attention
    from moba.kernels.gating import gate_select
    from moba.kernels.pooling import pool_blocks

    cfg = _cfg()
    b, s, hq, d = shape
    q, k, v, do = make_qkv((b, s, hq, d), torch.bfloat16, seed=0, n=4)
    if h_kv != hq:
        k, v = k[:, :, :h_kv].contiguous(), v[:, :, :h_kv].contiguous()
    cu = max_len = None
    if lens is not None:
        cu = torch.tensor([0] + torch.cumsum(torch.tensor(lens), 0).tolist(), dtype=torch.int32)
        max_len = max(lens)
    dev = "cuda"
    qg, kg, vg = (t.to(dev).requires_grad_(bwd) for t in (q, k, v))
    cug = None if cu is None else cu.to(dev)
    kbar = pool_blocks(kg.detach(), cfg, cu_seqlens=cug, max_seqlen=max_len)
    idx = gate_select(qg.detach(), kbar, cfg, cu_seqlens=cug, max_seqlen=max_len)
    out = moba_attention(qg, kg, vg, cfg, cu_seqlens=cug, max_seqlen=max_len)
    if bwd:
        out.backward(do.to(dev))
    torch.cuda.synchronize()
    kbar_ref = C.pool_blocks(k, BS, cu_seqlens=cu, max_seqlen=max_len)
    assert torch.equal(kbar.cpu(), kbar_ref), "pool differs from the C oracle"
    res = [t.detach().cpu() for t in (kbar, idx, out)]
    grads = [t.grad.cpu() for t in (qg, kg, vg)] if bwd else [None] * 3
    return q, k, v, do, cu, res, grads


def _blocks_for(length):
    nb = -(-length // BS)
    return sorted({nb - 1, max(0, nb - 4), nb // 2})


@pytest.mark.parametrize("name,shape,h_kv,bwd", [
    ("config2", (1, 65536, 4, 64), 4, False),
    ("config3", (1, 131072, 4, 64), 4, True),
    ("config4_gqa", (1, 32768, 32, 128), 8, True),
    ("headline_512k", (1, 524288, 4, 64), 4, True),
])
def test_full_size_padded(name, shape, h_kv, bwd):
    print(f"[full-size] {name} {shape} h_kv={h_kv} bwd={bwd}", flush=True)
    q, k, v, do, _, (kbar, idx, out), (dq, dk, dv) = _run(shape, h_kv, bwd)
    nb = kbar.shape[2]
    # GQA: the oracle's few heavy middle blocks would cost minutes on the
    # host; the tail blocks still cover the causal diagonal and past picks.
    blocks = [nb - 1, nb - 4] if h_kv != shape[2] else _blocks_for(shape[1])
    _check_sequence(name, q, k, v, do, kbar, idx, out, dq, dk, dv, bwd, blocks)


def test_full_size_varlen_config5():
    g = torch.Generator().manual_seed(0)
    lens = [int(x) // BS * BS for x in torch.randint(2048, 131073, (8,), generator=g)]
    total = sum(lens)
    print(f"[full-size] config5 varlen lens={lens} total={total}", flush=True)
    q, k, v, do, cu, (kbar, idx, out), (dq, dk, dv) = _run((1, total, 4, 64), 4, True, lens)
    for si in (0, len(lens) - 1):
        lo, hi = int(cu[si]), int(cu[si + 1])
        nbs = -(-(hi - lo) // BS)
        sl = slice(lo, hi)
        _check_sequence(f"config5 seq{si}", q[:, sl], k[:, sl], v[:, sl], do[:, sl],
                        kbar[si:si + 1, :, :nbs], idx[:, :, sl], out[:, sl],
                        dq[:, sl], dk[:, sl], dv[:, sl], True, _blocks_for(hi - lo))
