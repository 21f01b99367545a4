"""MoBA forward + backward throughput on one MI355X.

Metric: fwd & fwd+bwd ms at [1, S, 4, 64] bf16, block_size
128, top_k 8, S = 64K..512K, plus the fraction of the binding roofline.

A step is one training pass of the hot path on one batch of synthetic input:
`moba_attention(q, k, v).backward(dO)` -- pool, gate, CSC transpose, attend,
merge, delta, backward, dQ reduce -- with q, k, v, dO i.i.d. N(0, 1) already
resident in HBM. The headline workload is S = 524288 (the north star's
target size); the JSON line also carries the fwd and fwd+bwd sweep over
S = 64K..512K beside the reference's published H100 numbers.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--seq S]
       [--no-sweep] [--no-cpu]
       python bench.py --summarize-counters OUT.json DB... [--command CMD]
"""

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "moba-triton_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

import torch  # noqa: E402

HEADS, HEAD_DIM, BLOCK, TOPK = 4, 64, 128, 8
SWEEP = (65536, 131072, 262144, 524288)
# Reference Triton backend on H100.
H100_FWD_MS = {65536: 1.492, 131072: 3.942, 262144: 11.609, 524288: 38.164}
H100_FWDBWD_MS = {65536: 2.658, 131072: 6.181, 262144: 16.076, 524288: 47.046}
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
# HBM traffic per launch from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs,
# scaled by the same counters' reading for a plain copy of known size.
TRAFFIC_FILE = ROOT / "profiles" / "traffic_fwd_bwd_S524288.json"
# SQ / GRBM counters per kernel from rocprofv3 --pmc runs of this script
# (`--summarize-counters` writes it); the bench line reports the MFMA, VALU
# and LDS utilisation they give beside the algorithmic figures.
COUNTERS_FILE = ROOT / "profiles" / "counters_fwd_bwd_S524288.json"
# MI355X: 8 XCDs x 32 CUs x 4 SIMDs. GRBM_GUI_ACTIVE arrives summed over the
# XCDs, so GUI / 8 is the dispatch's clock count.
XCDS, CUS, SIMDS_PER_CU = 8, 256, 4
# Stage -> the kernel that dominates it (name as rocprofv3 reports it).
STAGE_KERNEL = {
    "pool": "pool_kernel", "gate": "gate_mfma_kernel", "csc": "det_scatter_kernel",
    "attend": "attend_mfma_kernel", "combine": "combine_kernel", "delta": "delta_kernel",
    "bwd": "bwd_mfma_kernel", "dq_reduce": "dq_reduce_kernel",
}


def algorithmic_bytes(s, b=1, hq=HEADS, hkv=HEADS, d=HEAD_DIM, k=TOPK, e=2):
    """Bytes each stage must move at minimum, per call (the per-unit figures
    of the design's traffic model times the units of one launch)."""
    n, nkv = b * hq * s, b * hkv * s
    return {
        "pool": nkv * d * e,
        "gate": n * d * e + 4 * n * k,
        "csc": 20 * n * k,
        "attend": k * n * d * e + 2 * nkv * d * e + 12 * n * k + n * k * d * e + 8 * n * k,
        "combine": n * k * d * e + 8 * n * k + n * d * e + 4 * n,
        "delta": 2 * n * d * e + 4 * n,
        "bwd": 2 * k * n * d * e + 8 * k * n + 4 * nkv * d * e + k * n * d * e + 12 * n * k,
        "dq_reduce": k * n * d * e + 4 * n * k + n * d * e,
    }


def gate_flops(s, hq=HEADS, d=HEAD_DIM, bs=BLOCK):
    """MFMA work of the gate per call: one D-long dot per (query, strictly
    past block) pair, padded to whole 32-block tiles as the kernel runs it."""
    pairs = 0
    for t0 in range(0, s, 128):       # 128 queries share one tile horizon
        hz = min(t0 + 127, s - 1) // bs
        pairs += 128 * ((hz + 31) // 32) * 32
    return 2 * d * pairs * hq


def _short_kernel(name):
    """`void moba::gate_mfma_kernel<...>(...)` -> `gate_mfma_kernel`."""
    return name.split("<")[0].split("(")[0].replace("void ", "").split("::")[-1]


def summarize_counters(out_path, dbs, command):
    """Reduces rocprofv3 `--pmc` databases (rocpd SQLite, one per counter
    pass) to per-kernel averages per dispatch plus derived utilisation:

    - mfma_busy = SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs x clocks)
    - valu_busy = SQ_ACTIVE_INST_VALU / (256 CUs x clocks)
    - lds_busy = SQ_LDS_IDX_ACTIVE / (256 CUs x clocks), of which
      lds_bank_conflict_frac = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE
    - waves_per_simd = 4 x SQ_WAVE_CYCLES (quad-cycles) / (1024 x clocks)
    - per-wave instruction counts (SQ_INSTS_* / SQ_WAVES)
    with clocks = GRBM_GUI_ACTIVE / 8 (the counter is summed over the XCDs).
    These are rocprofv3's own MfmaUtil / VALUBusy / LdsUtil definitions.
    """
    import collections
    import sqlite3

    sums = collections.defaultdict(lambda: collections.defaultdict(list))
    durs = collections.defaultdict(list)
    for db in dbs:
        con = sqlite3.connect(db)
        q = "select kernel_name, counter_name, value, duration, dispatch_id from counters_collection"
        seen = set()
        for kname, cname, val, dur, did in con.execute(q):
            k = _short_kernel(kname)
            sums[k][cname].append(float(val))
            if (db, did) not in seen:
                seen.add((db, did))
                durs[k].append(float(dur))
        con.close()
    kernels = {}
    for k, cs in sums.items():
        avg = {c: sum(v) / len(v) for c, v in cs.items()}
        row = {"dispatches": len(durs[k]), "avg_duration_us": round(sum(durs[k]) / len(durs[k]) / 1e3, 2),
               "counters": {c: round(v, 1) for c, v in sorted(avg.items())}}
        clk = avg.get("GRBM_GUI_ACTIVE", 0.0) / XCDS
        d = {}
        if clk > 0:
            simd_clk, cu_clk = clk * CUS * SIMDS_PER_CU, clk * CUS
            if "SQ_VALU_MFMA_BUSY_CYCLES" in avg:
                d["mfma_busy"] = avg["SQ_VALU_MFMA_BUSY_CYCLES"] / simd_clk
            if "SQ_ACTIVE_INST_VALU" in avg:
                d["valu_busy"] = avg["SQ_ACTIVE_INST_VALU"] / cu_clk
            if "SQ_LDS_IDX_ACTIVE" in avg:
                d["lds_busy"] = avg["SQ_LDS_IDX_ACTIVE"] / cu_clk
                if avg["SQ_LDS_IDX_ACTIVE"] > 0:
                    d["lds_bank_conflict_frac"] = avg.get("SQ_LDS_BANK_CONFLICT", 0.0) / avg["SQ_LDS_IDX_ACTIVE"]
            if "SQ_WAVE_CYCLES" in avg:  # quad-cycles summed over SIMDs
                d["waves_per_simd"] = 4 * avg["SQ_WAVE_CYCLES"] / simd_clk
            d["clock_ghz"] = clk / (row["avg_duration_us"] * 1e3)
        waves = avg.get("SQ_WAVES")
        if waves:
            for c in ("SQ_INSTS_VALU", "SQ_INSTS_SALU", "SQ_INSTS_LDS", "SQ_INSTS_MFMA",
                      "SQ_INSTS_VMEM_RD", "SQ_INSTS_VMEM_WR"):
                if c in avg:
                    d[c.replace("SQ_INSTS_", "insts_per_wave_").lower()] = avg[c] / waves
        row["derived"] = {n: round(v, 4) for n, v in d.items()}
        kernels[k] = row
    doc = {"command": command, "workload": "fwd+bwd [1,524288,4,64] bf16 bs128 k8",
           "note": "averages per dispatch; one rocprofv3 --pmc pass per database",
           "kernels": kernels}
    Path(out_path).write_text(json.dumps(doc, indent=1) + "\n")
    print(f"wrote {out_path}: {sorted(kernels)}")


def _pmc_per_kernel(db, counter):
    """{short kernel name: [(grid, value per dispatch), ...]} of one --pmc database."""
    import collections
    import sqlite3

    out = collections.defaultdict(list)
    con = sqlite3.connect(db)
    q = ("select kernel_name, counter_name, value, grid_size, dispatch_id "
         "from counters_collection")
    for kname, cname, val, grid, _ in con.execute(q):
        if cname == counter:
            out[_short_kernel(kname)].append((int(grid), float(val)))
    con.close()
    return out


def summarize_traffic(out_path, fetch_db, write_db, copy_fetch_db, copy_write_db, command):
    """HBM bytes per launch from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs
    of the headline workload, scaled by what the same counters read for a
    plain 1 GiB device copy (`--copy-probe`): hbm = FETCH KiB * 1024 * (copy
    bytes / copy FETCH bytes) + WRITE KiB * 1024 * (copy bytes / copy WRITE
    bytes). Per kernel, the average over its dispatches at the grid it has
    at the headline size (the largest grid it ran with)."""
    copy_bytes = 1 << 30

    def copy_kib(db, counter):  # the probe's copy dispatches (not its fill)
        vs = [v for k, d in _pmc_per_kernel(db, counter).items() if "copyBuffer" in k for _, v in d]
        return sum(vs) / len(vs)

    cf, cw = copy_kib(copy_fetch_db, "FETCH_SIZE"), copy_kib(copy_write_db, "WRITE_SIZE")
    ff, wf = copy_bytes / (cf * 1024), copy_bytes / (cw * 1024)
    fetch, write = _pmc_per_kernel(fetch_db, "FETCH_SIZE"), _pmc_per_kernel(write_db, "WRITE_SIZE")
    kernels = {}
    for k in sorted(set(fetch) & set(write)):
        if not k.strip() or "copyBuffer" in k:  # torch's own kernels, not the path's
            continue
        grid = max(g for g, _ in fetch[k])
        fv = [v for g, v in fetch[k] if g == grid]
        wv = [v for g, v in write[k] if g == grid]
        if not fv or not wv:
            continue
        fk, wk = sum(fv) / len(fv), sum(wv) / len(wv)
        kernels[k] = {"kernel": k, "seq_len": 524288, "grid": grid, "fetch_kib": round(fk, 1),
                      "write_kib": round(wk, 1),
                      "hbm_bytes_per_launch": int(fk * 1024 * ff + wk * 1024 * wf)}
    doc = {"workload": "fwd+bwd [1,524288,4,64] bf16, block_size 128, top_k 8 (bench.py defaults)",
           "commands": command.split(" ;; ") if command else [],
           "calibration": {"copy_bytes_each_way": copy_bytes, "copy_fetch_kib": round(cf, 4),
                           "copy_write_kib": round(cw, 4), "fetch_factor": round(ff, 4),
                           "write_factor": round(wf, 4),
                           "note": "hbm_bytes = FETCH_SIZE KiB * 1024 * fetch_factor + WRITE_SIZE "
                                   "KiB * 1024 * write_factor, per dispatch (average over the "
                                   "dispatches at the kernel's largest grid)"},
           "kernels": kernels}
    Path(out_path).write_text(json.dumps(doc, indent=1) + "\n")
    print(f"wrote {out_path}: {sorted(kernels)}")


def summarize_trace(out_path, db, command, bench_log):
    """Markdown table of a rocprofv3 --kernel-trace database: per kernel
    the calls, total and average duration over the whole run, plus the
    bench line's step time and per-stage times when its log is given."""
    import collections
    import sqlite3

    con = sqlite3.connect(db)
    agg = collections.defaultdict(list)
    for name, dur in con.execute("select name, duration from kernels"):
        agg[name].append(dur / 1e3)
    con.close()
    total = sum(sum(v) for v in agg.values())
    line = None
    if bench_log:
        for ln in Path(bench_log).read_text().splitlines():
            if ln.startswith("{"):
                line = json.loads(ln)
    out = ["# Kernel trace: bench.py default run (fwd+bwd, S=524288, plus the S=64K..512K sweep)", "",
           "Command (on the MI355X box, from the repo root):", "", "```", command, "```", "",
           "Read from the run's rocpd database (`kernels` view). Durations are GPU kernel times over "
           "the whole run (warm-up, timed steps, per-stage timing, the sweep, the hierarchical-gate "
           "probe, the offset-key step and the other BASELINE configurations)."]
    if line:
        out += ["", f"Bench line of the same run: `ms_per_step` = {line['ms_per_step']}; per-stage "
                "HIP-event medians (ms): " + ", ".join(f"{n} {r['ms']}" for n, r in
                                                        line["stages"].items()) + "."]
    out += ["", "| kernel | calls | total ms | avg us | % |", "|---|---:|---:|---:|---:|"]
    for name, v in sorted(agg.items(), key=lambda x: -sum(x[1])):
        nm = name if len(name) <= 110 else name[:107] + "..."
        out.append(f"| `{nm}` | {len(v)} | {sum(v) / 1e3:.3f} | {sum(v) / len(v):.1f} | "
                   f"{100 * sum(v) / total:.1f} |")
    Path(out_path).write_text("\n".join(out) + "\n")
    print(f"wrote {out_path}")


def make_inputs(s, dev, seed=0):
    g = torch.Generator(device=dev).manual_seed(seed)
    shape = (1, s, HEADS, HEAD_DIM)
    return [torch.randn(shape, generator=g, device=dev, dtype=torch.bfloat16) for _ in range(4)]


def timed(fn, reps, warmup):
    """Median and min of per-call device time (ms), events on the current stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        b.synchronize()
        times.append(a.elapsed_time(b))
    times.sort()
    return times[len(times) // 2], times[0]


def stage_times(s, dev, reps=5):
    """Per-stage device time (ms) of one fwd+bwd, each stage timed alone."""
    from moba.config import MoBAConfig
    from moba.kernels.gating import gate_select
    from moba.kernels.moba_bwd import bwd_kernel, compute_delta, reduce_dq
    from moba.kernels.moba_fwd import attend_partials, combine_partials
    from moba.kernels.pooling import pool_blocks
    from moba.kernels.routing import build_csc_from_indices
    from moba import _lib

    cfg = MoBAConfig(block_size=BLOCK, top_k=TOPK)
    q, k, v, do = make_inputs(s, dev)
    st = {}
    kbar = pool_blocks(k, cfg)
    st["pool"] = timed(lambda: pool_blocks(k, cfg), reps, 1)[0]
    idx = gate_select(q, kbar, cfg)
    st["gate"] = timed(lambda: gate_select(q, kbar, cfg), reps, 1)[0]
    index = build_csc_from_indices(idx, kbar.shape[2], cfg, num_kv_heads=HEADS)
    st["csc"] = timed(lambda: build_csc_from_indices(idx, kbar.shape[2], cfg,
                                                     num_kv_heads=HEADS), reps, 1)[0]
    parts = attend_partials(q, k, v, cfg, index)
    st["attend"] = timed(lambda: attend_partials(q, k, v, cfg, index, partials=parts),
                         reps, 1)[0]
    out, lse = combine_partials(*parts, q.dtype, return_lse=True)
    st["combine"] = timed(lambda: combine_partials(*parts, q.dtype, return_lse=True),
                          reps, 1)[0]
    st["delta"] = timed(lambda: compute_delta(out, do), reps, 1)[0]
    lse_delta = compute_delta(out, do, lse)
    dk, dv = torch.empty_like(k), torch.empty_like(v)
    dq_part = torch.empty((1, HEADS, s, TOPK, HEAD_DIM), device=dev, dtype=q.dtype)

    def bwd():
        bwd_kernel(do, q, k, v, lse_delta, cfg, index, dk, dv, dq_part)

    st["bwd"] = timed(bwd, reps, 1)[0]
    st["dq_reduce"] = timed(lambda: reduce_dq(dq_part, parts[0], q.dtype), reps, 1)[0]
    return st


def other_configs(dev, reps=5):
    """BASELINE.json configs 4 and 5 (config 3 is the sweep's 128K row):
    fwd and fwd+bwd device time of `moba_attention`, bf16, block 128, top-k 8.
    Config 4: GQA S=32768, Hq=32, Hkv=8, D=128. Config 5: 8 sequences of
    lengths U[2048, 131072] (seeded), rounded down to multiples of 128,
    packed (~512K tokens), H=4, D=64."""
    from moba.config import MoBAConfig
    from moba.kernels.attention import moba_attention
    from moba.kernels.moba_fwd import moba_forward

    cfg = MoBAConfig(block_size=BLOCK, top_k=TOPK)
    out = []
    g = torch.Generator().manual_seed(0)
    lens = [int(x) // BLOCK * BLOCK for x in torch.randint(2048, 131073, (8,), generator=g)]
    cases = [("config4_gqa", (1, 32768, 32, 128), 8, None),
             ("config5_varlen", (1, sum(lens), 4, 64), 4, lens)]
    for name, (b, s, hq, d), hkv, ln in cases:
        gd = torch.Generator(device=dev).manual_seed(0)
        q = torch.randn((b, s, hq, d), generator=gd, device=dev, dtype=torch.bfloat16)
        k, v = (torch.randn((b, s, hkv, d), generator=gd, device=dev, dtype=torch.bfloat16)
                for _ in range(2))
        do = torch.randn_like(q)
        kw = {}
        if ln is not None:
            cu = torch.tensor([0] + torch.cumsum(torch.tensor(ln), 0).tolist(), dtype=torch.int32,
                              device=dev)
            kw = {"cu_seqlens": cu, "max_seqlen": max(ln)}
        fwd = timed(lambda: moba_forward(q, k, v, cfg, **kw), reps, 2)[0]
        qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))

        def step():
            qq.grad = kk.grad = vv.grad = None
            moba_attention(qq, kk, vv, cfg, **kw).backward(do)

        fb = timed(step, reps, 2)[0]
        ab = algorithmic_bytes(s, b=b, hq=hq, hkv=hkv, d=d)
        ab_fwd = sum(ab[x] for x in ("pool", "gate", "csc", "attend", "combine"))
        ab_all = sum(ab.values())
        row = {"config": name, "shape": [b, s, hq, d], "heads_kv": hkv,
               "fwd_ms": round(fwd, 4), "fwd_bwd_ms": round(fb, 4),
               "tokens_per_s_fwd_bwd": round(s / (fb * 1e-3), 1),
               # the same traffic model as the headline roofline, at this shape
               "alg_bytes_fwd": ab_fwd, "alg_bytes_fwd_bwd": ab_all,
               "hbm_frac_fwd": round(ab_fwd / (fwd * 1e-3) / (HBM_PEAK_GBS * 1e9), 4),
               "hbm_frac_fwd_bwd": round(ab_all / (fb * 1e-3) / (HBM_PEAK_GBS * 1e9), 4)}
        if ln is not None:
            row["seq_lens"] = ln
        out.append(row)
        del q, k, v, do, qq, kk, vv
        torch.cuda.empty_cache()
    return out


def hierarchical_gate(s, dev, configs=((16, 8), (4, 8)), reps=5):
    """The opt-in hierarchical gate (`MoBAConfig.gate_group` / `gate_open`)
    beside the exact gate at S: device time of `gate_select` and recall --
    the share of the exact gate's strictly-past selections it keeps -- on the
    bench's i.i.d. keys (the worst case for any hierarchy) and on keys with
    positional locality (a random walk along the sequence plus unit noise),
    the two cases of the reference's `docs/gate-hierarchical-measurements.md`.
    Also the exact gate's own time on those keys and on keys that share one
    per-channel offset (3 offset + unit noise, as trained keys carry), whose
    block representatives nearly coincide so that many scores tie once
    rounded: `exact_gate_ms_by_keys`."""
    from moba.config import MoBAConfig
    from moba.kernels.gating import gate_select
    from moba.kernels.pooling import pool_blocks

    g = torch.Generator(device=dev).manual_seed(1)
    shape = (1, s, HEADS, HEAD_DIM)
    q = torch.randn(shape, generator=g, device=dev, dtype=torch.bfloat16)
    k_iid = torch.randn(shape, generator=g, device=dev, dtype=torch.bfloat16)
    walk = torch.randn(shape, generator=g, device=dev).mul_(0.05).cumsum_(1)
    k_walk = (walk + torch.randn(shape, generator=g, device=dev)).to(torch.bfloat16)
    del walk
    k_offset = (3.0 * torch.randn((1, 1, HEADS, HEAD_DIM), generator=g, device=dev)
                + torch.randn(shape, generator=g, device=dev)).to(torch.bfloat16)
    exact_cfg = MoBAConfig(block_size=BLOCK, top_k=TOPK)
    own = (torch.arange(s, device=dev) // BLOCK).view(1, 1, s, 1)

    def recall(sel, ref):
        ref_ok = (ref >= 0) & (ref != own)
        hit = (sel.unsqueeze(-1) == ref.unsqueeze(-2)).any(-2) & ref_ok
        return float(hit.sum()) / max(1.0, float(ref_ok.sum()))

    kbars = {"iid": pool_blocks(k_iid, exact_cfg), "walk": pool_blocks(k_walk, exact_cfg)}
    exact = {n: gate_select(q, kb, exact_cfg) for n, kb in kbars.items()}
    out = {"exact_gate_ms": round(timed(lambda: gate_select(q, kbars["iid"], exact_cfg),
                                        reps, 1)[0], 4), "configs": []}
    kb_offset = pool_blocks(k_offset, exact_cfg)
    del k_offset
    out["exact_gate_ms_by_keys"] = {
        n: round(timed(lambda: gate_select(q, kb, exact_cfg), reps, 1)[0], 4)
        for n, kb in (("iid", kbars["iid"]), ("walk", kbars["walk"]), ("offset", kb_offset))}
    for group, opened in configs:
        cfg = MoBAConfig(block_size=BLOCK, top_k=TOPK, gate_group=group, gate_open=opened)
        row = {"gate_group": group, "gate_open": opened,
               "gate_ms": round(timed(lambda: gate_select(q, kbars["iid"], cfg), reps, 1)[0], 4)}
        for n, kb in kbars.items():
            row["recall_" + n] = round(recall(gate_select(q, kb, cfg), exact[n]), 4)
        out["configs"].append(row)
    return out


def offset_key_step(s, dev, steps=5, warmup=2):
    """The whole fwd+bwd step (ms, wall clock between synchronizations, as the
    headline) on keys that share one per-channel offset (3 offset + unit
    noise, as trained keys carry): the gate's hardest distribution, beside
    the headline's i.i.d. keys. q, v, dO as the headline."""
    from moba.config import MoBAConfig
    from moba.kernels.attention import moba_attention

    cfg = MoBAConfig(block_size=BLOCK, top_k=TOPK)
    q, k, v, do = make_inputs(s, dev)
    g = torch.Generator(device=dev).manual_seed(2)
    k = (3.0 * torch.randn((1, 1, HEADS, HEAD_DIM), generator=g, device=dev)
         + torch.randn(k.shape, generator=g, device=dev)).to(torch.bfloat16)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))

    def step():
        qq.grad = kk.grad = vv.grad = None
        moba_attention(qq, kk, vv, cfg).backward(do)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    return round((time.perf_counter() - t0) * 1e3 / steps, 4)


def attainment(q, k, v, cfg, s, fwd_ms):
    """The reference's headline ratio (`bench/suite.py:1-12, 549-583`): the
    forward speedup over dense causal attention (torch SDPA, fused kernels
    only, via the `sdpa_dense` backend) divided by the speedup the sparsity
    pattern makes available (1 / `sparsity_ratio`)."""
    from implementations import get_backend
    from moba.sparsity import sparsity_ratio

    ceiling = 1.0 / sparsity_ratio(s, cfg)
    out = {"speedup_ceiling": round(ceiling, 2), "dense_fwd_ms": None,
           "speedup_vs_dense_fwd": None, "attainment_fwd": None}
    dense = get_backend("sdpa_dense")
    try:
        ms = timed(lambda: dense.forward(q, k, v, cfg), 2 if s >= 262144 else 5, 1)[0]
    except RuntimeError as exc:
        out["dense_note"] = str(exc)[:120]
        return out
    out.update(dense_fwd_ms=round(ms, 3), speedup_vs_dense_fwd=round(ms / fwd_ms, 2),
               attainment_fwd=round(ms / fwd_ms / ceiling, 4))
    return out


def sweep(dev, seqs, reps=5):
    from moba.config import MoBAConfig
    from moba.kernels.attention import moba_attention
    from moba.kernels.moba_fwd import moba_forward

    cfg = MoBAConfig(block_size=BLOCK, top_k=TOPK)
    rows = []
    for s in seqs:
        q, k, v, do = make_inputs(s, dev)
        fwd = timed(lambda: moba_forward(q, k, v, cfg), reps, 2)[0]
        qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))

        def step():
            qq.grad = kk.grad = vv.grad = None
            moba_attention(qq, kk, vv, cfg).backward(do)

        fb = timed(step, reps, 2)[0]
        row = {"seq_len": s, "fwd_ms": round(fwd, 4), "fwd_bwd_ms": round(fb, 4),
               "h100_ref_fwd_ms": H100_FWD_MS.get(s),
               "h100_ref_fwd_bwd_ms": H100_FWDBWD_MS.get(s),
               "speedup_fwd": round(H100_FWD_MS[s] / fwd, 2) if s in H100_FWD_MS else None,
               "speedup_fwd_bwd": round(H100_FWDBWD_MS[s] / fb, 2)
               if s in H100_FWDBWD_MS else None}
        row.update(attainment(q, k, v, cfg, s, fwd))
        rows.append(row)
        del q, k, v, do, qq, kk, vv
        torch.cuda.empty_cache()
    return rows


def cpu_baseline(s, rows_sample=1024):
    """The oracle on the host: pool (C), gate (C) for a sample of query rows
    at full length S, and the float32 sparse-gather attention fwd+bwd (torch
    autograd) for those rows. Reported as query tokens per second."""
    from oracle import c_oracle
    from oracle import naive as O
    from types import SimpleNamespace

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    os.environ.setdefault("OMP_NUM_THREADS", str(threads))
    ocfg = SimpleNamespace(block_size=BLOCK, top_k=TOPK, always_select_current=True,
                           top_k_includes_current=True, tie_break_low_index=True)
    g = torch.Generator().manual_seed(0)
    shape = (1, s, HEADS, HEAD_DIM)
    q, k, v, do = (torch.randn(shape, generator=g) for _ in range(4))
    rows = torch.linspace(0, s - 1, rows_sample).long()
    t0 = time.perf_counter()
    kbar = c_oracle.pool_blocks(k, BLOCK)
    qs = q[:, rows].contiguous()
    # gate the sampled rows against the full-length representatives
    n = kbar.shape[2]
    idx = torch.full((1, HEADS, rows_sample, TOPK), -1, dtype=torch.int32)
    qs_f = qs.double()
    kb = kbar.double()
    for i, t in enumerate(rows.tolist()):
        own = t // BLOCK
        take = min(TOPK - 1, own)
        sc = torch.einsum("hd,hnd->hn", qs_f[0, i], kb[0, :, :own]).float()
        if take > 0:
            top = torch.sort(sc, dim=-1, descending=True, stable=True).indices[:, :take]
            sel = torch.sort(top, dim=-1).values
            idx[0, :, i, :take] = sel.int()
        idx[0, :, i, take] = own
    qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))
    full_idx = torch.full((1, HEADS, s, TOPK), -1, dtype=torch.int32)
    full_idx[:, :, rows] = idx
    out, _ = O.moba_attention_sparse(qg, kg, vg, full_idx, BLOCK, rows=rows)
    out.backward(do[:, rows])
    dt = time.perf_counter() - t0
    return {"value": round(rows_sample / dt, 2), "unit": "query tokens/s (fwd+bwd, 4 heads)",
            "cores": threads, "kind": "port",
            "sample": f"{rows_sample} evenly spaced query rows of the S={s} fwd+bwd workload "
                      f"(C-oracle pool + exact gate for those rows, fp32 sparse-gather "
                      f"attention fwd+bwd via torch autograd); {dt:.1f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--seq", type=int, default=524288)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-hier", action="store_true",
                    help="skip the opt-in hierarchical gate's timing and recall")
    ap.add_argument("--cpu-rows", type=int, default=16384)
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a plain 1 GiB device copy (HBM counter calibration)")
    ap.add_argument("--summarize-counters", nargs="+", metavar=("OUT_JSON", "DB"),
                    help="reduce rocprofv3 --pmc databases to OUT_JSON and exit (no GPU)")
    ap.add_argument("--command", default="", help="with --summarize-counters: the "
                    "profiling command, recorded in OUT_JSON")
    ap.add_argument("--summarize-traffic", nargs=5,
                    metavar=("OUT_JSON", "FETCH_DB", "WRITE_DB", "COPY_FETCH_DB", "COPY_WRITE_DB"),
                    help="reduce FETCH_SIZE / WRITE_SIZE databases to OUT_JSON and exit (no GPU)")
    ap.add_argument("--summarize-trace", nargs=2, metavar=("OUT_MD", "DB"),
                    help="reduce a --kernel-trace database to OUT_MD and exit (no GPU)")
    ap.add_argument("--bench-log", default="", help="with --summarize-trace: the run's output")
    args = ap.parse_args()
    if args.summarize_traffic:
        summarize_traffic(*args.summarize_traffic, args.command)
        return
    if args.summarize_trace:
        summarize_trace(*args.summarize_trace, args.command, args.bench_log)
        return
    if args.summarize_counters:
        summarize_counters(args.summarize_counters[0], args.summarize_counters[1:], args.command)
        return
    if args.copy_probe:
        x = torch.empty(1 << 29, dtype=torch.int16, device="cuda:0").fill_(1)
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes_each_way": x.numel() * x.element_size()}))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    from moba.config import MoBAConfig
    from moba.kernels.attention import moba_attention

    dev = torch.device("cuda:0")
    s = args.seq
    cfg = MoBAConfig(block_size=BLOCK, top_k=TOPK)
    q, k, v, do = make_inputs(s, dev)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))

    def step():
        qq.grad = kk.grad = vv.grad = None
        moba_attention(qq, kk, vv, cfg).backward(do)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = wall * 1e3 / args.steps
    print(f"[bench] S={s} fwd+bwd {ms:.3f} ms/step", file=sys.stderr, flush=True)
    del qq, kk, vv
    torch.cuda.empty_cache()

    stages = stage_times(s, dev)
    ab = algorithmic_bytes(s)
    gf = gate_flops(s)
    stage_rows = {}
    for n, t in stages.items():
        row = {"ms": round(t, 4), "kernel": STAGE_KERNEL[n],
               "alg_GBps": round(ab[n] / (t * 1e-3) / 1e9, 1),
               "hbm_frac": round(ab[n] / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        if n == "gate":
            row["mfma_TFLOPs"] = round(gf / (t * 1e-3) / 1e12, 1)
            row["mfma_frac"] = round(gf / (t * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)
        stage_rows[n] = row
    if COUNTERS_FILE.exists():
        ck = json.loads(COUNTERS_FILE.read_text()).get("kernels", {})
        for n, row in stage_rows.items():
            dv = ck.get(STAGE_KERNEL[n], {}).get("derived", {})
            for key in ("mfma_busy", "valu_busy", "lds_busy"):
                if key in dv:
                    row["rocprof_" + key] = dv[key]
    print(f"[bench] stages {stage_rows}", file=sys.stderr, flush=True)
    dom = max(stages, key=stages.get)
    traffic = None
    if TRAFFIC_FILE.exists():
        tr = json.loads(TRAFFIC_FILE.read_text()).get("kernels", {}).get(STAGE_KERNEL[dom])
        if tr and tr.get("seq_len") == s:
            traffic = tr["hbm_bytes_per_launch"]
    if dom == "gate":
        achieved = gf / (stages[dom] * 1e-3) / 1e12
        roof = {"bound": "mfma", "kernel": STAGE_KERNEL[dom], "achieved": round(achieved, 1),
                "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": traffic,
                "algorithmic": gf}
    else:
        achieved = ab[dom] / (stages[dom] * 1e-3) / 1e9
        roof = {"bound": "hbm", "kernel": STAGE_KERNEL[dom], "achieved": round(achieved, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "algorithmic": ab[dom]}
    total_alg = sum(ab.values())
    rows = [] if args.no_sweep else sweep(dev, SWEEP)
    hier = None if args.no_hier else hierarchical_gate(s, dev)
    torch.cuda.empty_cache()
    offset_ms = None if args.no_hier else offset_key_step(s, dev)
    torch.cuda.empty_cache()
    configs = [] if args.no_sweep else other_configs(dev)
    torch.cuda.empty_cache()
    cpu = None if args.no_cpu else cpu_baseline(s, args.cpu_rows)
    tokens = s  # query tokens per step (batch 1)
    line = {
        "metric": "fwd & fwd+bwd ms at [1,S,4,64] bs128 k8, S=64K..512K; % MFMA/HBM peak",
        "value": round(tokens / (ms * 1e-3), 1),
        "unit": "tokens/s (fwd+bwd, S=%d)" % s,
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": round(H100_FWDBWD_MS[s] / ms, 3) if s in H100_FWDBWD_MS else None,
        "dtype": "bf16", "data": "synthetic (q, k, v, dO i.i.d. N(0,1), seed 0)",
        "config": {"workload": "moba_fwd_bwd", "batch": 1, "seq_len": s, "heads_q": HEADS,
                   "heads_kv": HEADS, "head_dim": HEAD_DIM, "block_size": BLOCK,
                   "top_k": TOPK, "causal": True},
        "roofline": roof,
        "step_roofline": {"alg_bytes": total_alg,
                          "alg_GBps": round(total_alg / (ms * 1e-3) / 1e9, 1),
                          "frac": round(total_alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
        "stages": stage_rows,
        # The same step on keys with a shared per-channel offset (the gate's
        # hardest distribution), beside ms_per_step on i.i.d. keys.
        "step_ms_by_keys": {"iid": round(ms, 4), "offset": offset_ms},
        "sweep": rows,
        "hierarchical_gate": hier,
        "other_configs": configs,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
