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
Tolerance (bf16, the north star's bars made scale-aware for gradients that
sum over many queries): max-abs <= 2e-2 * max(1, max|truth|) and
mean-abs <= 2e-3 * max(1, mean|truth|).
"""

import pytest
import torch

from conftest import make_qkv, oracle_cfg
from oracle import c_oracle as C
from oracle import naive as O
from tolerance import assert_selection_matches

pytestmark = pytest.mark.gpu

BS, TOPK = 128, 8
MAX_GATHER_BYTES = 256 << 20  # float64 gather budget of one oracle chunk


def _cfg():
    from moba.config import MoBAConfig
    return MoBAConfig(block_size=BS, top_k=TOPK)


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


def _oracle_rows(qd, kd, vd, do, idx, rows):
    """Float64 sparse oracle over `rows` in bounded chunks; returns the
    outputs of those rows and accumulates q/k/v grads of (out * dO).sum()."""
    h, d = qd.shape[2], qd.shape[3]
    per_row = h * idx.shape[-1] * BS * d * 8 * 3
    chunk = max(1, MAX_GATHER_BYTES // per_row)
    outs = []
    for lo in range(0, rows.numel(), chunk):
        r = rows[lo:lo + chunk]
        o, _ = O.moba_attention_sparse(qd, kd, vd, idx, BS, rows=r)
        (o * do[:, r].double()).sum().backward()
        outs.append(o.detach())
    return torch.cat(outs, dim=1)


def _check_sequence(name, q, k, v, do, kbar, idx, out, dq, dk, dv, bwd, blocks):
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
    qd, kd, vd = (t.double().requires_grad_(True) for t in (q, k, v))
    o_ref = _oracle_rows(qd, kd, vd, do, idx, rows)
    _bars(out[:, rows], o_ref, f"{name} O rows")
    if not bwd:
        return
    _bars(dq[:, rows], qd.grad[:, rows], f"{name} dQ rows")
    # dK / dV of sampled blocks, from every query that selected them
    hit = (idx[..., None] == torch.tensor(blocks)).any(-1).any(-1).any(1)[0]   # [L]
    users = torch.nonzero(hit).flatten()
    kd2, vd2 = (t.double().requires_grad_(True) for t in (k, v))
    _oracle_rows(q.double(), kd2, vd2, do, idx, users)
    keys = torch.cat([torch.arange(b * BS, min((b + 1) * BS, length)) for b in blocks])
    _bars(dk[:, keys], kd2.grad[:, keys], f"{name} dK blocks {blocks}")
    _bars(dv[:, keys], vd2.grad[:, keys], f"{name} dV blocks {blocks}")


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
