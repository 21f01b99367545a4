"""Writes the golden fixtures in this directory from the reference oracle.

Run in the build container only (the reference tree is not present on GPU
boxes):  python tests/golden/make_golden.py [/root/reference]

It loads three reference modules by file path -- `src/moba/config.py`,
`src/moba/gqa.py`, `src/moba/naive.py` -- without executing the package
`__init__` (which would pull in the Triton kernels), calls the reference's
own `pool_blocks_naive`, `gate_select_naive`, `moba_selection` and
`moba_attention_naive` on seeded inputs, and stores inputs digests and
outputs as compressed `.npz` data. Nothing of the reference's source is
stored; only the vectors.

Inputs follow the reference's `make_qkv` scheme (`tests/conftest.py:83-98`):
one CPU `torch.Generator` seeded once, q, k, v drawn in that order.
"""

import hashlib
import importlib.util
import sys
import types
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def load_reference(root: Path):
    pkg = types.ModuleType("moba")
    pkg.__path__ = [str(root / "src" / "moba")]
    sys.modules["moba"] = pkg
    mods = {}
    for name in ("config", "gqa", "naive"):
        spec = importlib.util.spec_from_file_location(
            f"moba.{name}", root / "src" / "moba" / f"{name}.py")
        mod = importlib.util.module_from_spec(spec)
        sys.modules[f"moba.{name}"] = mod
        spec.loader.exec_module(mod)
        mods[name] = mod
    return mods


def make_qkv(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(shape, generator=g, dtype=dtype) for _ in range(3))


def digest(*ts):
    h = hashlib.sha256()
    for t in ts:
        h.update(t.contiguous().view(torch.uint8).numpy().tobytes())
    return h.hexdigest()


def bits(t):
    """Raw storage bits of a tensor, as a numpy integer array."""
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.contiguous().view(torch.int16).numpy()
    if t.dtype == torch.float32:
        return t.contiguous().view(torch.int32).numpy()
    return t.numpy()


def sel_indices(mask, slots):
    n = mask.shape[-1]
    ids = torch.arange(n).expand_as(mask)
    key = torch.where(mask, ids, torch.full_like(ids, n)).sort(-1).values
    key = key[..., :slots]
    return torch.where(key < n, key, torch.full_like(key, -1)).to(torch.int16).numpy()


def main(root: Path):
    ref = load_reference(root)
    Cfg = ref["config"].MoBAConfig
    naive = ref["naive"]
    out = {}

    # -- gate cases: bf16 selection + kbar, reference GATE_SWEEP shapes -------
    gate_cases = [
        # (name, shape, block_size, top_k, dtype, seed, h_kv)
        ("g_s4096_d64_b128_k8", (1, 4096, 4, 64), 128, 8, torch.bfloat16, 0, 4),
        ("g_s2048_d128_b64_k8", (1, 2048, 4, 128), 64, 8, torch.bfloat16, 0, 4),
        ("g_s2048_d64_b32_k4", (1, 2048, 4, 64), 32, 4, torch.bfloat16, 0, 4),
        ("g_s1024_d128_b32_k8_b2", (2, 1024, 4, 128), 32, 8, torch.bfloat16, 0, 4),
        ("g_s4096_d64_b128_k12", (1, 4096, 4, 64), 128, 12, torch.bfloat16, 1, 4),
        ("g_s16384_d64_b32_k64", (1, 16384, 1, 64), 32, 64, torch.bfloat16, 2, 1),
        ("g_gqa_s2048_d128_b64_k4", (1, 2048, 8, 128), 64, 4, torch.bfloat16, 3, 2),
        ("g_s4096_d64_b128_k8_f16", (1, 4096, 4, 64), 128, 8, torch.float16, 0, 4),
        ("g_s1000_d64_b128_k8_tail", (1, 1000, 2, 64), 128, 8, torch.bfloat16, 4, 2),
    ]
    for name, shape, bs, tk, dt, seed, h_kv in gate_cases:
        cfg = Cfg(block_size=bs, top_k=tk, dtype=dt)
        b, s, h, d = shape
        q, k, _ = make_qkv(shape, dt, seed)
        if h_kv != h:
            k = k[:, :, :h_kv].contiguous()
        kbar = naive.pool_blocks_naive(k, cfg)
        sel = naive.gate_select_naive(q, kbar, cfg)
        out[f"{name}__digest"] = np.array(digest(q, k))
        out[f"{name}__kbar_bits"] = bits(kbar)
        out[f"{name}__idx"] = sel_indices(sel, tk)
        out[f"{name}__meta"] = np.array([b, s, h, d, bs, tk, seed, h_kv,
                                         {torch.bfloat16: 0, torch.float16: 1,
                                          torch.float32: 2}[dt]])

    # -- forced ties (tests/test_gate.py:95-120) -----------------------------
    cfg = Cfg(block_size=64, top_k=2, dtype=torch.bfloat16)
    q, k, _ = make_qkv((1, 512, 1, 64), torch.bfloat16, 0)
    kbar = naive.pool_blocks_naive(k, cfg)
    kbar[:] = kbar[:, :, :1, :]
    sel = naive.gate_select_naive(q, kbar, cfg)
    out["ties__digest"] = np.array(digest(q, k))
    out["ties__kbar_bits"] = bits(kbar)
    out["ties__idx"] = sel_indices(sel, 2)

    # -- varlen selection (tests/test_varlen.py:20-24) ------------------------
    cu = torch.tensor([0, 80, 128, 192, 212], dtype=torch.int32)
    cfg = Cfg(block_size=16, top_k=3, dtype=torch.bfloat16)
    q, k, _ = make_qkv((1, 212, 2, 64), torch.bfloat16, 5)
    sel = naive.moba_selection(q, k, cfg, cu_seqlens=cu)
    out["varlen__digest"] = np.array(digest(q, k))
    out["varlen__idx"] = sel_indices(sel, 3)
    out["varlen__cu"] = cu.numpy()

    # -- non-default flags (config.py:21-61) ---------------------------------
    for tag, kw in [("nocur", dict(always_select_current=False)),
                    ("excl", dict(top_k_includes_current=False))]:
        cfg = Cfg(block_size=32, top_k=3, dtype=torch.bfloat16, **kw)
        q, k, _ = make_qkv((1, 512, 2, 64), torch.bfloat16, 6)
        sel = naive.moba_selection(q, k, cfg)
        out[f"{tag}__digest"] = np.array(digest(q, k))
        out[f"{tag}__idx"] = sel_indices(sel, 4)

    # -- attention: config 1 (fp32 [1,4096,4,64] bs128 k8), rows subset -------
    cfg = Cfg(block_size=128, top_k=8, dtype=torch.float32)
    q, k, v = make_qkv((1, 4096, 4, 64), torch.float32, 0)
    o = naive.moba_attention_naive(q, k, v, cfg, query_chunk=512)
    sel = naive.moba_selection(q, k, cfg)
    rows = torch.arange(0, 4096, 16)
    out["cfg1__digest"] = np.array(digest(q, k, v))
    out["cfg1__rows"] = rows.numpy()
    out["cfg1__out_rows"] = o[:, rows].numpy()
    out["cfg1__out_sum"] = np.array([o.double().sum().item(),
                                     o.double().square().sum().item()])
    out["cfg1__idx"] = sel_indices(sel, 8)

    # -- attention in float64, small shapes, full outputs ---------------------
    att_cases = [
        ("a64_gqa", (1, 256, 4, 32), 2, 32, 3, 7),
        ("a64_tail", (1, 200, 2, 32), 2, 64, 2, 8),
    ]
    for name, shape, h_kv, bs, tk, seed in att_cases:
        cfg = Cfg(block_size=bs, top_k=tk, dtype=torch.float64)
        q, k, v = make_qkv(shape, torch.float64, seed)
        k = k[:, :, :h_kv].contiguous()
        v = v[:, :, :h_kv].contiguous()
        o = naive.moba_attention_naive(q, k, v, cfg)
        out[f"{name}__digest"] = np.array(digest(q, k, v))
        out[f"{name}__out"] = o.numpy()

    # -- packed attention in float64 ------------------------------------------
    cfg = Cfg(block_size=16, top_k=3, dtype=torch.float64)
    q, k, v = make_qkv((1, 212, 2, 32), torch.float64, 9)
    o = naive.moba_attention_naive(q, k, v, cfg, cu_seqlens=cu)
    out["avarlen__digest"] = np.array(digest(q, k, v))
    out["avarlen__out"] = o.numpy()

    np.savez_compressed(HERE / "reference_oracle.npz", **out)
    print("wrote", HERE / "reference_oracle.npz", len(out), "arrays")


if __name__ == "__main__":
    main(Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference"))
