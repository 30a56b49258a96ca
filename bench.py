"""Headline benchmark: MoC memory cross-attention fwd+bwd at the paper shape.

Workload: B=8 sequences x L=1024 tokens, d=768, 12 query /
12 KV heads (head_dim 64), bank of 262,208 tokens = 4,097 chapters x 64
(1 shared + 4,096 routed), sequence-level routing top-k=64, routed scaling
2.5 -> every sequence attends to 65 x 64 = 4,160 memory keys.  bf16 tensors,
fp32 accumulation, router in fp32.  One step = router forward + memory layer
forward + backward of everything (dh, dWq..dWo, dbank rows, router weight
and bias grads through the omega chain) for one batch of synthetic inputs
already resident in HBM.

Prints one JSON line.  `value` = tokens/s of the whole step; the per-kernel
roofline object is measured with HIP events around each launch in the timed
region; `cpu_baseline` times the CPU oracle (the PyTorch-CPU restatement of
the reference's path, fp32) on a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

MFMA_BF16_PEAK_TFLOPS = 2500.0
HBM_PEAK_GBS = 8000.0

CFG = dict(B=8, L=1024, d=768, H=12, HK=12, C=4097, T=64, S=1, k=64, scale=2.5)


def algorithmic_flops(cfg, unique_chapters=None):
    """FLOP counts (GEMM = 2MNK; attention = 4 * queries * H * keys * Dh; fwd+bwd = 3x fwd)."""
    B, L, d, H, HK, T, S, k = (cfg[x] for x in ("B", "L", "d", "H", "HK", "T", "S", "k"))
    Dh = d // H
    ntok = B * L
    keys = (S + k) * T
    q = 2.0 * ntok * d * d
    kv = 2.0 * B * keys * d * (2 * HK * Dh)
    attn = 4.0 * ntok * H * keys * Dh
    o = 2.0 * ntok * d * d
    fwd = q + kv + attn + o
    out = dict(q=q, kv=kv, attn=attn, o=o, fwd=fwd, step=3.0 * fwd)
    if unique_chapters is not None:
        out["kv_project_launch"] = 2.0 * unique_chapters * T * d * (2 * HK * Dh)
    out["xattn_fwd_launch"] = attn
    # algorithmic backward attention work split by kernel: dq launch = dQ product (1x of the
    # 2 fwd products' size / 2), dkv launch = dK and dV products; recomputed S / dP are not credited.
    out["xattn_bwd_dq_launch"] = attn / 2.0
    out["xattn_bwd_dkv_launch"] = attn
    return out


def build_inputs(dev, dtype, cfg, seed=0):
    import torch
    from memory_amd.model import RoutedMemoryLayer

    torch.manual_seed(seed)
    B, L, d, H, C, T = (cfg[x] for x in ("B", "L", "d", "H", "C", "T"))
    h = torch.randn(B, L, d, device=dev, dtype=dtype)
    bank = (torch.randn(C * T, d, device=dev, dtype=torch.float32) * 0.02).to(dtype)
    layer = RoutedMemoryLayer(d, H, C, T, cfg["k"], num_shared_chapters=cfg["S"],
                              routed_scaling_factor=cfg["scale"], num_kv_heads=cfg["HK"], wo_init_zero=False)
    with torch.no_grad():
        for lin in (layer.memory_attn.q_proj, layer.memory_attn.k_proj, layer.memory_attn.v_proj,
                    layer.memory_attn.o_proj):
            lin.weight.normal_(0.0, 0.02)
        layer.router.router.weight.normal_(0.0, 0.02)
        layer.router.router.bias.zero_()
    layer = layer.to(dev)
    for lin in (layer.memory_attn.q_proj, layer.memory_attn.k_proj, layer.memory_attn.v_proj,
                layer.memory_attn.o_proj):
        lin.to(dtype)
    torch.manual_seed(1)
    dout = torch.randn(B, L, d, device=dev, dtype=dtype)
    h.requires_grad_(True)
    bank.requires_grad_(True)
    return layer, h, bank, dout


def run_step(layer, h, bank, dout):
    h.grad = None
    bank.grad = None
    for p in layer.parameters():
        p.grad = None
    out, _ = layer(h, bank, return_losses=False)
    out.backward(dout)
    return out


def cpu_baseline(cfg, budget_s=20.0):
    """Oracle (PyTorch-CPU restatement of the reference path) fwd+bwd in fp32 on one sequence."""
    import torch
    import oracle as O

    ncores = len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)
    g = torch.Generator().manual_seed(0)
    Bs = 1
    L, d, H, C, T, S, k = (cfg[x] for x in ("L", "d", "H", "C", "T", "S", "k"))
    h = torch.randn(Bs, L, d, generator=g)
    bank = torch.randn(C * T, d, generator=g) * 0.02
    Wr = torch.randn(C, d, generator=g) * 0.02
    br = torch.zeros(C)
    Wq, Wk, Wv, Wo = (torch.randn(d, d, generator=g) * 0.02 for _ in range(4))
    dO = torch.randn(Bs, L, d, generator=g)
    leaves = [t.requires_grad_(True) for t in (h, bank, Wr, br, Wq, Wk, Wv, Wo)]

    def once():
        for t in leaves:
            t.grad = None
        out = O.sequence_memory_layer(*leaves, H=H, HK=cfg["HK"], C=C, T=T, S=S, top_k=k,
                                      routed_scale=cfg["scale"])
        out.backward(dO)

    t0 = time.perf_counter()
    once()                              # warm-up
    warm = time.perf_counter() - t0
    iters = max(3, min(10, int(budget_s / max(warm, 1e-3))))
    times = []
    for _ in range(iters):
        t0 = time.perf_counter()
        once()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"value": Bs * L / med, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "affinity_cores": ncores, "torch_threads": torch.get_num_threads(), "cpu_model": cpu_model(),
            "sample": f"oracle sequence_memory_layer fwd+bwd fp32, 1 sequence x {L} tokens at the full paper shape "
                      f"(d={d}, H={H}, bank {C * T} rows, k={k}); 1 warm-up, median of {iters} iterations "
                      f"({med * 1e3:.0f} ms each); tokens/s of that sequence"}


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo, as lscpu reports it)."""
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.lower().startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


PROBE_BYTES = 256 << 20
# entry point -> device kernel whose HBM traffic the counter passes measured
# entry point / native-layer stage -> the device kernel its roofline figures are about
TRAFFIC_KERNELS = {"moc_xattn_bwd_dkv": "xattn_bwd_dkv_kernel<bf16>", "moc_xattn_fwd": "xattn_fwd_kernel<bf16>",
                   "moc_xattn_bwd_dq": "xattn_bwd_dq_kernel<bf16>", "moc_kv_project": "kv_project_wide_kernel",
                   "moc_decode_partial": "sparse_fwd_unit_kernel", "moc_sparse_bwd": "sparse_bwd_unit_kernel",
                   "moc_bank_adamw": "bank_adamw_kernel"}


def kernel_sources():
    """Device kernel name (without template arguments) -> the HIP source that defines it, read
    from the `__global__` declarations under memory_amd/csrc."""
    import glob
    import re
    out = {}
    for path in sorted(glob.glob(os.path.join(ROOT, "memory_amd", "csrc", "*.hip"))):
        with open(path) as f:
            text = f.read()
        for n in re.findall(r"__global__(?:\s+__launch_bounds__\([^)]*\))?\s+void\s+(\w+)\s*\(", text):
            out.setdefault(n, os.path.basename(path))
    return out


def source_sha(kernel: str):
    """First 16 hex digits of the SHA-256 of the HIP source ``kernel`` is built from."""
    import hashlib
    src = kernel_sources().get(kernel.split("<")[0])
    if src is None:
        return None
    path = os.path.join(ROOT, "memory_amd", "csrc", src)
    if not os.path.exists(path):
        return None
    with open(path, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()[:16]


def profile_value(workload: str, key: str, kern: str, kind: str = "traffic"):
    """A per-kernel figure from a committed counter summary (profiles/<kind>_<workload>.md, lines
    `<key> <kernel> <value> <source sha16>`), returned only while the kernel's HIP source still
    hashes to the recorded value: (value or None, note)."""
    path = os.path.join(ROOT, "profiles", f"{kind}_{workload}.md")
    if kern is None or not os.path.exists(path):
        return None, "no profile"
    with open(path) as f:
        for ln in f:
            parts = ln.strip().strip("`").split()
            if len(parts) >= 3 and parts[0] == key and parts[1] == kern:
                sha = parts[3] if len(parts) > 3 else None
                cur = source_sha(kern)
                if sha is None or sha != cur:
                    return None, f"stale: {os.path.basename(path)} measured source {sha}, current {cur}"
                return float(parts[2]), f"profiles/{kind}_{workload}.md (source {sha})"
    return None, "kernel not in profile"


def measured_traffic(workload, entry):
    """HBM bytes per launch of `entry`'s kernel from the committed counter summary
    (profiles/traffic_<workload>.md), or None when absent or measured on another source."""
    v, note = profile_value(workload, "traffic_bytes", TRAFFIC_KERNELS.get(entry))
    return (None if v is None else int(v)), note


XCDS, SIMDS, CUS = 8, 1024, 256   # MI355X: GRBM_GUI_ACTIVE sums the 8 XCDs' counts


_MANGLED_TYPES = {"DF16b": "bf16", "f": "f32", "d": "f64", "i": "i32", "l": "i64", "b": "bool"}


def _short_kernel(name: str) -> str:
    """`kernel<template args>` from a rocprofv3 kernel name, mangled (`_ZN3moc...`) or demangled
    (`void moc::...::name<2, 0>(...)`); the arguments tell instantiations apart."""
    import re
    if name.startswith("_ZN"):
        i, parts = 3, []
        while i < len(name) and name[i].isdigit():
            m = re.match(r"\d+", name[i:])
            n = int(m.group(0))
            i += len(m.group(0))
            parts.append(name[i:i + n])
            i += n
        base, args = parts[-1] if parts else name[:48], []
        if i < len(name) and name[i] == "I":
            i += 1
            while i < len(name) and name[i] != "E":
                lit = re.match(r"L(DF16b|[a-z])(-?\d+)E", name[i:])
                if lit:
                    args.append(lit.group(2))
                    i += len(lit.group(0))
                    continue
                for code, t in _MANGLED_TYPES.items():
                    if name.startswith(code, i):
                        args.append(t)
                        i += len(code)
                        break
                else:
                    break
        return base + (f"<{','.join(args)}>" if args else "")
    m = re.search(r"(\w+)(<[^()]*>)?\(", name)
    if not m:
        return name[:48]
    args = (m.group(2) or "").replace(" ", "").replace("float", "f32")
    return m.group(1) + args


def traffic_summary(fetch_csv, write_csv):
    """HBM bytes per launch and kernel from two rocprofv3 --pmc runs (FETCH_SIZE, then
    WRITE_SIZE; counter_collection.csv, KiB per dispatch), each scaled by what the same counter
    reads for the plain PROBE_BYTES device copy (`--traffic-probe`, `__amd_rocclr_copyBuffer`)
    of the same run.  Prints a markdown table and the machine-readable lines bench.py reads back
    (tied to the kernel source's hash)."""
    import csv
    from collections import defaultdict

    def read(path, counter):
        per = defaultdict(list)
        with open(path) as f:
            for r in csv.DictReader(f):
                if r["Counter_Name"] == counter:
                    per[_short_kernel(r["Kernel_Name"])].append(float(r["Counter_Value"]))
        return per

    fe, wr = read(fetch_csv, "FETCH_SIZE"), read(write_csv, "WRITE_SIZE")
    probe = "__amd_rocclr_copyBuffer"
    if probe not in fe or probe not in wr:
        raise SystemExit(f"traffic summary: no {probe} dispatch (run with --traffic-probe)")
    kib = PROBE_BYTES / 1024.0
    f_scale, w_scale = kib / max(fe[probe]), kib / max(wr[probe])
    rows, lines = [], []
    for k in sorted(set(fe) & set(wr)):
        if source_sha(k) is None:   # runtime copies, torch and rocprim kernels
            continue
        f, w = sum(fe[k]) / len(fe[k]), sum(wr[k]) / len(wr[k])
        nbytes = (f * f_scale + w * w_scale) * 1024.0
        rows.append(f"| `{k}` | {len(fe[k])} | {f:.1f} | {w:.1f} | {nbytes / 1e6:.1f} MB |")
        sha = source_sha(k)
        if sha is not None:
            lines.append(f"    traffic_bytes {k} {nbytes:.0f} {sha}")
    head = (f"Probe copy ({PROBE_BYTES} bytes read and written): FETCH_SIZE {max(fe[probe]):.1f} KiB, "
            f"WRITE_SIZE {max(wr[probe]):.1f} KiB, so bytes = FETCH_SIZE x {f_scale:.4f} x 1024 + "
            f"WRITE_SIZE x {w_scale:.4f} x 1024.\n\n"
            "| kernel | launches | FETCH_SIZE (KiB) | WRITE_SIZE (KiB) | HBM bytes / launch (scaled) |\n"
            "|---|---:|---:|---:|---:|")
    return head + "\n" + "\n".join(rows) + "\n\nMachine-readable (read by bench.py):\n\n" + "\n".join(lines)


def stats_summary(path):
    """Markdown table of a rocprofv3 --kernel-trace --stats kernel_stats.csv with the kernels named
    as `kernel<template args>` and the HIP source each one is built from."""
    import csv
    src = kernel_sources()
    rows = ["| kernel | source | calls | avg (us) | total (ms) | % |", "|---|---|---:|---:|---:|---:|"]
    with open(path) as f:
        for r in csv.DictReader(f):
            k = _short_kernel(r["Name"])
            if len(k) > 72:
                k = k[:69] + "..."
            rows.append(f"| `{k}` | {src.get(k.split('<')[0], '-')} | {r['Calls']} | "
                        f"{float(r['AverageNs']) / 1e3:.1f} | {float(r['TotalDurationNs']) / 1e6:.3f} | "
                        f"{float(r['Percentage']):.1f} |")
    return "\n".join(rows)


def pmc_summary(paths):
    """Per-kernel means of rocprofv3 --pmc counter_collection.csv files (several passes with
    different counters may be given): MFMA-busy, VALU-busy and co-issue fractions of the
    SIMD-cycles of a launch, LDS activity and conflicts, instructions per wave.  Prints a
    markdown table and the machine-readable lines bench.py reads back (tied to the kernel
    source's hash)."""
    import csv
    from collections import defaultdict
    per = defaultdict(lambda: defaultdict(dict))
    grid = {}
    for p in paths:
        with open(p) as f:
            for r in csv.DictReader(f):
                k = _short_kernel(r["Kernel_Name"])
                per[k][(p, r["Dispatch_Id"])][r["Counter_Name"]] = float(r["Counter_Value"])
                grid[k] = int(r["Grid_Size"])
    rows, lines = [], []
    for k in sorted(per):
        if source_sha(k) is None:   # runtime copies, torch and rocprim kernels
            continue
        acc = defaultdict(list)
        for c in per[k].values():
            for n, v in c.items():
                acc[n].append(v)
        a = {n: sum(v) / len(v) for n, v in acc.items()}
        cyc = a.get("GRBM_GUI_ACTIVE", 0.0) / XCDS
        if cyc <= 0:
            continue
        waves = max(1, grid[k] // 64)
        f = lambda n, scale=1.0, den=SIMDS: (scale * a[n] / (den * cyc)) if n in a else None
        mb, vb = f("SQ_VALU_MFMA_BUSY_CYCLES"), f("SQ_ACTIVE_INST_VALU", 4.0)
        co, lds = f("SQ_VALU_MFMA_COEXEC_CYCLES"), f("SQ_LDS_IDX_ACTIVE", den=CUS)
        conf = (a["SQ_LDS_BANK_CONFLICT"] / a["SQ_LDS_IDX_ACTIVE"]) if a.get("SQ_LDS_IDX_ACTIVE") else None
        ipw = {n: a[n] / waves for n in ("SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_VALU_TRANS_F32", "SQ_INSTS_LDS",
                                          "SQ_INSTS_SALU") if n in a}
        fmt = lambda v: "-" if v is None else f"{v:.3f}"
        rows.append(f"| `{k}` | {len(per[k])} | {cyc / 2400:.1f} | {fmt(mb)} | {fmt(vb)} | {fmt(co)} | {fmt(lds)} | "
                    f"{fmt(conf)} | " + " / ".join(f"{ipw.get(n, 0):.0f}" for n in
                                                     ("SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_VALU_TRANS_F32",
                                                      "SQ_INSTS_LDS", "SQ_INSTS_SALU")) + " |")
        sha = source_sha(k)
        if sha is None:
            continue
        if mb is not None:
            lines.append(f"    mfma_busy {k} {mb:.4f} {sha}")
        if vb is not None:
            lines.append(f"    valu_busy {k} {vb:.4f} {sha}")
    head = ("| kernel | dispatches | us at 2.4 GHz (GRBM_GUI_ACTIVE / 8) | MFMA busy | VALU busy | MFMA+VALU co-issue | "
            "LDS active (per CU) | LDS conflicts / access | per wave: VALU (incl. MFMA) / MFMA / TRANS_F32 / LDS / SALU |\n"
            "|---|---:|---:|---:|---:|---:|---:|---:|---|")
    return head + "\n" + "\n".join(rows) + "\n\nMachine-readable (read by bench.py):\n\n" + "\n".join(lines)


def traffic_fields(workload, entry):
    v, note = measured_traffic(workload, entry)
    return {"traffic": v, "traffic_source": note}


def counter_fields(workload, entry):
    """The roofline kernel's MFMA-busy fraction (SQ_VALU_MFMA_BUSY_CYCLES over the SIMD-cycles of
    the launch) and VALU-busy fraction from the committed SQ counter summary
    (profiles/counters_<workload>.md), tied to the kernel's source like the traffic."""
    kern = TRAFFIC_KERNELS.get(entry)
    mb, note = profile_value(workload, "mfma_busy", kern, "counters")
    vb, _ = profile_value(workload, "valu_busy", kern, "counters")
    return {"mfma_busy": mb, "valu_busy": vb, "counters_source": note}


def kernel_table(events, steps):
    per = {}
    for name, pairs in events.items():
        durs = [a.elapsed_time(b) for a, b in pairs]
        per[name] = {"calls_per_step": len(pairs) / steps, "avg_ms": sum(durs) / len(durs),
                     "ms_per_step": sum(durs) / steps}
    return per


def stage_table(stages, steps):
    """Per-kernel table entries from the native layer's stage timing (moc_seq_layer_timing)."""
    return {n: {"calls_per_step": c / steps, "avg_ms": t / c, "ms_per_step": t / steps}
            for n, (t, c, _) in stages.items() if c}


def profile_pass(fn, steps):
    """Untimed pass with events around every entry point and every stage of the native layer
    (its kernels are launched from inside moc_seq_layer_fwd / _bwd): the per-kernel table."""
    import torch
    from memory_amd import _lib
    torch.cuda.synchronize()
    _lib.seq_stage_timing(None, steps)
    _lib.KERNEL_EVENTS, _lib.KERNEL_EVENTS_ONLY = {}, None
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    ev, _lib.KERNEL_EVENTS = _lib.KERNEL_EVENTS, None
    stages = stage_table(_lib.seq_stage_read(), steps)
    _lib.seq_stage_timing(None, 0)
    return {**kernel_table(ev, steps), **stages}, set(stages)


def timed(fn, steps, warmup, roofline_entry=None):
    """warmup untimed steps, an instrumented pass (per-kernel table), then exactly `steps`
    timed steps bracketed by synchronize; inside the timed region only the launches of
    the roofline kernel (given, or the one with the most time per step in the
    instrumented pass) carry events, so the step time is not inflated by per-launch
    markers.  Returns (ms per step, per-kernel table, roofline entry, its timed-region
    table entry)."""
    import torch
    from memory_amd import _lib
    for _ in range(warmup):
        fn()
    per, stage_names = profile_pass(fn, min(steps, 10))
    if roofline_entry is None and per:
        # the host calls of the native layer span many kernels: the roofline kernel is one of its stages
        kern = [n for n in per if not n.startswith("moc_seq_layer_")]
        roofline_entry = max(kern or per, key=lambda n: per[n]["ms_per_step"])
    is_stage = roofline_entry in stage_names
    torch.cuda.synchronize()
    if is_stage:
        _lib.seq_stage_timing([roofline_entry], steps)
    else:
        _lib.KERNEL_EVENTS, _lib.KERNEL_EVENTS_ONLY = {}, {roofline_entry}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    if is_stage:
        live = stage_table(_lib.seq_stage_read(), steps).get(roofline_entry)
        _lib.seq_stage_timing(None, 0)
    else:
        ev = _lib.KERNEL_EVENTS
        _lib.KERNEL_EVENTS, _lib.KERNEL_EVENTS_ONLY = None, None
        live = kernel_table(ev, steps).get(roofline_entry)
    return wall * 1e3 / steps, per, roofline_entry, live


# stages of the native layer launched on its side streams (moc_seq_layer_fwd's aux stream,
# moc_seq_layer_bwd's aux and fill streams)
SIDE_STREAM_STAGES = {"moc_weight_pack:wkv", "moc_rows_linear:q_proj", "moc_weight_pack:transposed",
                      "moc_linear_wgrad:o_proj", "moc_fill_zero:dbank", "moc_rows_linear:q_proj_dx",
                      "moc_linear_wgrad:q_proj", "moc_router_seq_bwd+linear_bwd+pool_bwd"}


C4 = dict(B=4, L=2048, d=768, H=12, HK=12, C=4097, T=64, S=1, k=16, scale=2.5)


def c4_flops(cfg):
    B, L, d, H, HK, C, T, S, k = (cfg[x] for x in ("B", "L", "d", "H", "HK", "C", "T", "S", "k"))
    ntok, Dh = B * L, d // H
    router = 2.0 * ntok * d * C
    q = o = 2.0 * ntok * d * d
    attn = 4.0 * ntok * H * (S + k) * T * Dh
    kv = 2.0 * (C - S) * T * d * (2 * HK * Dh) + 2.0 * S * T * d * (2 * HK * Dh)
    fwd = router + q + o + attn + kv
    return dict(router=router, q=q, o=o, attn=attn, kv=kv, fwd=fwd, step=3.0 * fwd)


def run_c4(args, losses_timing=True):
    import torch
    from memory_amd.model import TokenRoutedMemoryLayer
    cfg = dict(C4)
    dev = torch.device("cuda", 0)
    dtype = torch.bfloat16
    torch.manual_seed(0)
    B, L, d, H, C, T = (cfg[x] for x in ("B", "L", "d", "H", "C", "T"))
    h = torch.randn(B, L, d, device=dev, dtype=dtype, requires_grad=True)
    bank = (torch.randn(C * T, d, device=dev) * 0.02).to(dtype).requires_grad_(True)
    layer = TokenRoutedMemoryLayer(d, H, C, T, cfg["k"], num_shared_chapters=cfg["S"],
                                   routed_scaling_factor=cfg["scale"], weighted=True, kernel_version="v4",
                                   wo_init_zero=False).to(dev)
    with torch.no_grad():
        for lin in (layer.memory_attn.q_proj, layer.memory_attn.k_proj, layer.memory_attn.v_proj,
                    layer.memory_attn.o_proj):
            lin.weight.normal_(0.0, 0.02)
            lin.to(dtype)
        layer.router.router.weight.normal_(0.0, 0.02)
    torch.manual_seed(1)
    dout = torch.randn(B, L, d, device=dev, dtype=dtype)

    def step():
        h.grad = None
        bank.grad = None
        for p in layer.parameters():
            p.grad = None
        out, _ = layer(h, bank, return_losses=False)
        out.backward(dout)

    # distinct chapters of this batch's routing (per-launch bytes of the sparse backward)
    with torch.no_grad():
        idx, _, _ = layer.router.route_token_level(h.detach(), return_losses=False,
                                                   exclude_prefix_chapters=cfg["S"])
        n_chap = int(torch.unique(idx).numel())
    ms, per, _, live = timed(step, args.steps, args.warmup, "moc_sparse_bwd")
    losses = router_losses_timing(layer, h, cfg) if losses_timing else None
    fl = c4_flops(cfg)
    tflops = fl["step"] / (ms * 1e-3) / 1e12
    kernels = {n: {"avg_ms": round(v["avg_ms"], 4), "calls": v["calls_per_step"]}
               for n, v in sorted(per.items(), key=lambda kv: -kv[1]["ms_per_step"])}
    roofline = None
    if live:
        # sparse backward: K and V tiles of the selected (chapter, kv head) units read, their dK and
        # dV written, q and dO read and dq written once per (token, head)
        tile = 64 * 64 * 2
        unit_bytes = n_chap * cfg["HK"] * tile * 2 * 2
        row_bytes = B * L * H * 64 * 2 * 3
        alg = unit_bytes + row_bytes
        ach = alg / (live["avg_ms"] * 1e-3) / 1e9
        roofline = {"kernel": "moc_sparse_bwd", "bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4), **traffic_fields("c4", "moc_sparse_bwd"),
                    "avg_ms": round(live["avg_ms"], 4), "algorithmic_bytes": alg, "selected_chapters": n_chap}
    return {
        "metric": "token-level memory-xattn fwd+bwd tokens/s (B=4,L=2048,d=768,k=16,T=64)",
        "value": round(B * L / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "c4: token-level routed memory layer fwd+bwd (v4 MoE combine)", **cfg},
        "tflops": round(tflops, 2), "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
        "algorithmic_gflop_per_step": round(fl["step"] / 1e9, 1), "roofline": roofline, "kernels": kernels,
        **({"router_losses": losses} if losses is not None else {}),
    }


def router_losses_timing(layer, h, cfg, iters=20):
    """The router's auxiliary losses (router.py:197-260) at the token-level shape, forward +
    backward of their sum: the fused kernels against the same formulas as unfused torch ops
    (the reference's (rows, k, C) one-hot included), both on the GPU."""
    import torch
    import torch.nn.functional as F
    from memory_amd import ops
    C, k = cfg["C"], cfg["k"]
    with torch.no_grad():
        logits0 = ops.router_token_logits(h.detach(), layer.router.router.weight, layer.router.router.bias)
        idx = torch.topk(logits0[:, 1:], k, dim=-1).indices + 1

    def fused():
        z = logits0.detach().requires_grad_(True)
        v = ops.router_losses(z, idx, C)
        sum(v.values()).backward()

    def unfused():
        z = logits0.detach().requires_grad_(True)
        probs = torch.softmax(z, dim=-1)
        f = F.one_hot(idx, num_classes=C).float().sum(dim=1).mean(dim=0)
        lb = C * (f * probs.mean(dim=0)).sum()
        aux = F.mse_loss(probs.pow(2).mean(dim=0), torch.full((C,), 1.0 / C, device=z.device))
        zl = (torch.logsumexp(z, dim=-1) ** 2).mean()
        ent = -(probs * torch.log(probs.clamp_min(1e-12))).sum(dim=-1).mean()
        (lb + aux + zl + ent).backward()

    out = {"rows": int(logits0.shape[0]), "chapters": C, "k": k}
    for name, fn in (("fused_ms", fused), ("torch_ops_ms", unfused)):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(iters):
            fn()
        torch.cuda.synchronize()
        out[name] = round((time.perf_counter() - t0) * 1e3 / iters, 4)
    # the fused entry points' own GPU time (HIP events on the launch stream), outside the loop above
    from memory_amd import _lib as L
    L.KERNEL_EVENTS, L.KERNEL_EVENTS_ONLY = {}, {"moc_router_losses", "moc_router_losses_bwd"}
    try:
        for _ in range(iters):
            fused()
        torch.cuda.synchronize()
        ev = L.KERNEL_EVENTS
    finally:
        L.KERNEL_EVENTS, L.KERNEL_EVENTS_ONLY = None, None
    for n, key in (("moc_router_losses", "fused_fwd_kernels_ms"), ("moc_router_losses_bwd", "fused_bwd_kernels_ms")):
        pairs = ev.get(n, [])
        out[key] = round(sum(a.elapsed_time(b) for a, b in pairs) / max(1, len(pairs)), 4)
    return out


C5 = dict(B=64, d=768, H=12, HK=12, C=4097, T=64, S=1, k=64, scale=2.5, layers=4, prompt=512)


def run_c5(args):
    import torch
    from memory_amd.decode import DecodeRouting, DecodeStepGraph, MemoryDecodeCache, memory_decode_step
    from memory_amd.model import RoutedMemoryLayer
    cfg = dict(C5)
    dev = torch.device("cuda", 0)
    dtype = torch.bfloat16
    torch.manual_seed(0)
    B, d, H, HK, C, T = (cfg[x] for x in ("B", "d", "H", "HK", "C", "T"))
    bank = (torch.randn(C * T, d, device=dev) * 0.02).to(dtype)
    layers = []
    with torch.no_grad():
        prompt = torch.randn(B, cfg["prompt"], d, device=dev, dtype=dtype)
        for _ in range(cfg["layers"]):
            lay = RoutedMemoryLayer(d, H, C, T, cfg["k"], num_shared_chapters=cfg["S"],
                                    routed_scaling_factor=cfg["scale"], num_kv_heads=HK, wo_init_zero=False).to(dev)
            for lin in (lay.memory_attn.q_proj, lay.memory_attn.k_proj, lay.memory_attn.v_proj,
                        lay.memory_attn.o_proj):
                lin.weight.normal_(0.0, 0.02)
                lin.to(dtype)
            lay.router.router.weight.normal_(0.0, 0.02)
            idx_star, omega, _ = lay.route(prompt, return_losses=False)
            cache = MemoryDecodeCache(bank, lay.memory_attn.k_proj.weight, lay.memory_attn.v_proj.weight,
                                      num_chapters=C, tokens_per_chapter=T, num_kv_heads=HK, dtype=dtype)
            layers.append((lay, cache, DecodeRouting(idx_star, omega, C)))
        h_t = torch.randn(B, 1, d, device=dev, dtype=dtype)
    uniq = [r.unique_chapters() for _, _, r in layers]
    tile_bytes = 64 * 64 * 2 * HK * 2          # K + V of one chapter, all kv heads, bf16
    unique_bytes = sum(uniq) * tile_bytes
    per_seq_bytes = cfg["layers"] * B * (cfg["S"] + cfg["k"]) * tile_bytes

    def step():
        for lay, cache, routing in layers:
            memory_decode_step(lay.memory_attn, h_t, cache, routing)

    ms, per, _, dec = timed(step, args.steps, args.warmup, "moc_decode_partial")
    # the same step replayed from one captured HIP graph (the serving path for a fixed batch)
    graph = DecodeStepGraph([(lay.memory_attn, cache, routing) for lay, cache, routing in layers],
                            [h_t] * len(layers))
    # the token's hidden states sit in the graph's input buffers, as a serving loop writes them
    # (the graph was captured with h_t in them)
    for _ in range(args.warmup):
        graph.run(graph.static_in)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        graph.run(graph.static_in)
    torch.cuda.synchronize()
    graph_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    del graph
    # the same step when every layer re-routes at every token ("rolling" inference strategy,
    # window 128: window pooling, router logits, top-k + prepend, chapter plan, then the decode)
    from memory_amd.decode import DecodeRouter
    routers = [DecodeRouter(lay.router, num_chapters=C, num_shared_chapters=cfg["S"],
                            routed_scaling_factor=cfg["scale"], strategy="rolling", window_size=128)
               for lay, _, _ in layers]
    with torch.no_grad():
        for dr in routers:
            dr.prefill(prompt)

    def rerouted_step():
        for (lay, cache, _), dr in zip(layers, routers):
            memory_decode_step(lay.memory_attn, h_t, cache, dr.step(h_t))

    for _ in range(args.warmup):
        rerouted_step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        rerouted_step()
    torch.cuda.synchronize()
    rerouted_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    roofline = None
    if dec:
        ach = (unique_bytes / cfg["layers"]) / (dec["avg_ms"] * 1e-3) / 1e9
        roofline = {"kernel": "moc_decode_partial", "bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                    **traffic_fields("c5", "moc_decode_partial"),
                    "avg_ms": round(dec["avg_ms"], 4), "algorithmic_bytes": unique_bytes / cfg["layers"]}
    kernels = {n: {"avg_ms": round(v["avg_ms"], 4), "calls": v["calls_per_step"]}
               for n, v in sorted(per.items(), key=lambda kv: -kv[1]["ms_per_step"])}
    return {
        "metric": "memory-layer decode HBM GB/s (4 layers, B=64, k=64, T=64; unique selected K/V bytes)",
        "value": round(unique_bytes / (ms * 1e-3) / 1e9, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "c5: decode step through 4 memory layers sharing one bank", **cfg,
                   "unique_chapters_per_layer": uniq},
        "hbm_frac": round(unique_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "per_sequence_gbs": round(per_seq_bytes / (ms * 1e-3) / 1e9, 1),
        "tokens_per_s": round(B / (ms * 1e-3), 1),
        "roofline": roofline, "kernels": kernels,
        "graph_replay": {"ms_per_step": round(graph_ms, 4),
                         "gbs": round(unique_bytes / (graph_ms * 1e-3) / 1e9, 1),
                         "tokens_per_s": round(B / (graph_ms * 1e-3), 1)},
        "rerouted_rolling": {"ms_per_step": round(rerouted_ms, 4),
                             "tokens_per_s": round(B / (rerouted_ms * 1e-3), 1)},
    }


# training-run optimizer settings of the reference (configs/base_small_run2.yaml:111, :159-163)
BANK_OPT = dict(lr=6e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
MAX_GRAD_NORM = 1.0


def run_c3opt(args):
    """The config-3 memory layer's training step with the bank's optimizer: router + layer
    forward, backward, clip_grad_norm_ over the bank and the layer's parameters, AdamW on the
    fp32 bank (training/trainer.py:876-889).  Four batches are cycled so the routed chapters
    change between steps.  Variants:
      reference_style - the kernels read the fp32 bank, dense fp32 bank gradient,
                        torch.nn.utils.clip_grad_norm_ and foreach torch.optim.AdamW;
      bank_adamw      - BankAdamW: row-sparse bank gradient, exact lazy catch-up, bf16 mirror
                        read by the kernels (the value of this line);
      bank_adamw_dense - BankAdamW without row sparsity (dense gradient, one fused pass).
    Only the bank is stepped (the layer's own parameters are clipped but not updated), so
    every variant runs the same routing."""
    import torch
    from memory_amd.bank_optim import BankAdamW, clip_grad_norm_

    dev = torch.device("cuda", 0)
    dtype = torch.bfloat16
    cfg = dict(CFG)
    layer, h, _, dout = build_inputs(dev, dtype, cfg)
    B, L, C, T, d = cfg["B"], cfg["L"], cfg["C"], cfg["T"], cfg["d"]
    torch.manual_seed(2)
    bank0 = torch.randn(C * T, d, device=dev, dtype=torch.float32) * 0.02
    hs = [torch.randn(B, L, d, device=dev, dtype=dtype).requires_grad_(True) for _ in range(4)]
    with torch.no_grad():
        plans = [set(torch.unique(layer.route(x, return_losses=False)[0]).tolist()) for x in hs]
    elems = T * d
    step_bytes = [len(plans[i]) * elems * 30 + len(plans[i] - plans[i - 1]) * elems * 26 for i in range(4)]

    def make(kind):
        bank = torch.nn.Parameter(bank0.clone())
        if kind == "reference_style":
            opt = torch.optim.AdamW([bank], foreach=True, **BANK_OPT)
        else:
            opt = BankAdamW(bank, T, mirror_dtype=torch.bfloat16, row_sparse=(kind == "bank_adamw"), **BANK_OPT)
        params = [bank, *layer.parameters()]
        it = [0]

        def step():
            x = hs[it[0] % len(hs)]
            it[0] += 1
            x.grad = None
            for p in layer.parameters():
                p.grad = None
            out, _ = layer(x, bank, return_losses=False)
            out.backward(dout)
            if kind == "reference_style":
                torch.nn.utils.clip_grad_norm_(params, MAX_GRAD_NORM)
            else:
                clip_grad_norm_(params, MAX_GRAD_NORM)
            opt.step()
            opt.zero_grad()
        return step

    res = {}
    kinds = [k for k in ("reference_style", "bank_adamw_dense", "bank_adamw") if k in args.variants.split(",")]
    if "bank_adamw" not in kinds:
        raise SystemExit("--variants must include bank_adamw (the value of the c3opt line)")
    for kind in kinds:
        step = make(kind)
        entry = "moc_bank_adamw" if kind == "bank_adamw" else None
        ms, per, _, live = timed(step, args.steps, args.warmup, roofline_entry=entry)
        res[kind] = {"ms_per_step": round(ms, 4),
                     "kernels": {n: {"avg_ms": round(v["avg_ms"], 4), "calls": v["calls_per_step"]}
                                 for n, v in sorted(per.items(), key=lambda kv: -kv[1]["ms_per_step"])[:8]}}
        if kind == "bank_adamw":
            res[kind]["live"] = live
        torch.cuda.synchronize()
        del step
        torch.cuda.empty_cache()

    ms = res["bank_adamw"]["ms_per_step"]
    live = res["bank_adamw"].pop("live")
    roofline = None
    if live:
        # both launches of a step (catch-up of the plan's stale chapters, then the step of the
        # touched ones): algorithmic bytes per launch = the cycle's mean bytes per step / 2
        per_launch = sum(step_bytes) / len(step_bytes) / live["calls_per_step"]
        ach = per_launch / (live["avg_ms"] * 1e-3) / 1e9
        roofline = {"kernel": "moc_bank_adamw", "bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                    **traffic_fields("c3opt", "moc_bank_adamw"),
                    "avg_ms": round(live["avg_ms"], 4), "algorithmic_bytes": int(per_launch)}
    return {
        "metric": "memory-layer training step tokens/s incl. clip + bank AdamW (L=1024,d=768,k=64,T=64)",
        "value": round(B * L / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (four seeded batches cycled; N(0,0.02) fp32 bank)",
        "config": {"workload": "c3opt: config-3 memory layer fwd+bwd + clip_grad_norm_ + AdamW on the fp32 bank",
                   **{k: cfg[k] for k in ("B", "L", "d", "H", "C", "T", "S", "k")}, **BANK_OPT,
                   "max_grad_norm": MAX_GRAD_NORM,
                   "chapters_per_step": [len(p) for p in plans]},
        "variants": res,
        "roofline": roofline,
    }


def run_c3block(args):
    """The memory sublayer of a transformer block at config 3 (memory_block.py:549-558):
    routing on the block input, memory_layernorm (RMSNorm, eps 1e-5 as configs/base_small_run2.yaml:40),
    memory cross-attention over the routed chapters, o_proj and the residual add; forward +
    backward.  Variants:
      reference_style - the reference's RMSNorm module as torch ops (memory_block.py:26-28), then
                        o_proj and a separate residual add;
      norm_kernel     - MemorySublayer with the norm as one HIP row kernel writing bf16 ahead of the
                        q projection, the residual as the o_proj GEMM's accumulator input;
      fused           - MemorySublayer with the norm folded into the q projection's GEMM
                        (ops.norm_linear) and the residual as above (the value of this line)."""
    import torch
    from memory_amd import ops
    from memory_amd.memory_block import MemorySublayer

    dev = torch.device("cuda", 0)
    dtype = torch.bfloat16
    cfg = dict(CFG)
    layer, h, bank, dout = build_inputs(dev, dtype, cfg)
    B, L, d, C, T = cfg["B"], cfg["L"], cfg["d"], cfg["C"], cfg["T"]
    sub = MemorySublayer(d, cfg["H"], cfg["HK"], use_rms_norm=True, norm_eps=1e-5, wo_init_zero=False).to(dev)
    sub.memory_attn = layer.memory_attn            # the bf16 projections of the c3 layer
    norm_w = sub.memory_layernorm.weight

    def state(x):
        idx_star, omega, _ = layer.route(x, return_losses=False)
        return {"bank": bank, "chapter_indices": idx_star, "chapter_weights": omega, "num_chapters": C,
                "tokens_per_chapter": T}

    def ref_rms(x):
        rms = torch.sqrt(x.pow(2).mean(-1, keepdim=True) + 1e-5)
        return x / rms * norm_w

    def step_ref():
        h.grad = bank.grad = norm_w.grad = None
        for p in layer.parameters():
            p.grad = None
        x = ref_rms(h).to(dtype)
        pre = layer.memory_attn.attention_preproj(x, routed_memory_state=state(h))
        out = h + ops.linear(pre, layer.memory_attn.o_proj.weight)
        out.backward(dout)

    def step_sub(fuse):
        def step():
            h.grad = bank.grad = norm_w.grad = None
            for p in layer.parameters():
                p.grad = None
            sub.fuse_norm = fuse
            out = sub(h, routed_memory_state=state(h))
            out.backward(dout)
        return step

    res = {}
    for kind, fn in (("reference_style", step_ref), ("norm_kernel", step_sub(False)), ("fused", step_sub(True))):
        ms, per, _, _ = timed(fn, args.steps, args.warmup)
        res[kind] = {"ms_per_step": round(ms, 4),
                     "kernels": {n: {"avg_ms": round(v["avg_ms"], 4), "calls": v["calls_per_step"]}
                                 for n, v in sorted(per.items(), key=lambda kv: -kv[1]["ms_per_step"])
                                 if n in ("moc_row_norm_fwd", "moc_row_norm_bwd", "moc_rows_linear_norm",
                                          "moc_norm_fold_weight")}}
    ms = res["fused"]["ms_per_step"]
    return {
        "metric": "memory sublayer fwd+bwd tokens/s incl. memory_layernorm + residual (L=1024,d=768,k=64,T=64)",
        "value": round(B * L / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded N(0,1) hidden states, random-init)",
        "config": {"workload": "c3block: memory_layernorm + routed memory cross-attention + residual, fwd+bwd",
                   **{k: cfg[k] for k in ("B", "L", "d", "H", "C", "T", "S", "k")}, "norm": "rms", "norm_eps": 1e-5},
        "variants": res,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", choices=["c3", "c4", "c5", "c3opt", "c3block"], default="c3")
    ap.add_argument("--gpus", type=int, default=1)
    # steady state: the c3 step measured 0.867-0.883 ms over 20 steps after 5 warm-up steps and
    # 0.841-0.843 ms over 100 after 20 (clocks and caches settle over the first tens of ms)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--variants", default="reference_style,bank_adamw_dense,bank_adamw",
                    help="c3opt: which optimizer variants to run (comma-separated)")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--no-losses-timing", action="store_true",
                    help="c4: skip the router-loss comparison (fused kernels vs unfused torch ops) that "
                         "follows the timed steps, so that a kernel trace holds the step's kernels only")
    ap.add_argument("--headline-only", action="store_true",
                    help="c3: skip the c5 decode and c4 token-level lines that ride along the headline")
    ap.add_argument("--pmc-summary", nargs="+", metavar="CSV",
                    help="print the per-kernel summary of rocprofv3 --pmc counter_collection.csv files and exit")
    ap.add_argument("--stats-summary", metavar="STATS_CSV",
                    help="print a rocprofv3 --stats kernel_stats.csv as a markdown table and exit")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="print the per-kernel HBM bytes of a FETCH_SIZE and a WRITE_SIZE "
                         "counter_collection.csv (runs made with --traffic-probe) and exit")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run one plain 256 MiB device copy before the warmup: the reference kernel "
                         "that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes")
    args = ap.parse_args()
    if args.pmc_summary:
        print(pmc_summary(args.pmc_summary))
        return
    if args.stats_summary:
        print(stats_summary(args.stats_summary))
        return
    if args.traffic_summary:
        print(traffic_summary(*args.traffic_summary))
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); "
              "the path shards by sequence with no exchange in the forward, see DESIGN.md", file=sys.stderr)
        sys.exit(2)

    if args.traffic_probe:
        import torch
        src = torch.ones(PROBE_BYTES // 4, device="cuda:0", dtype=torch.float32)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    if args.workload != "c3":
        run = {"c4": lambda a: run_c4(a, losses_timing=not a.no_losses_timing), "c5": run_c5, "c3opt": run_c3opt,
               "c3block": run_c3block}[args.workload]
        print(json.dumps(run(args)), flush=True)
        return

    import torch
    from memory_amd import _lib

    dev = torch.device("cuda", 0)
    dtype = torch.bfloat16
    cfg = dict(CFG)
    layer, h, bank, dout = build_inputs(dev, dtype, cfg)
    run_step(layer, h, bank, dout)
    torch.cuda.synchronize()

    # unique chapters of this batch (for the per-launch FLOP count of the projection)
    with torch.no_grad():
        idx_star, _, _ = layer.route(h, return_losses=False)
        n_unique = int(torch.unique(idx_star).numel())

    # the roofline kernel is the attention backward's dK/dV kernel (the largest main-stream stage;
    # stages on the side streams overlap it, so their event spans include time shared with it)
    ms, per_kernel, dom, live = timed(lambda: run_step(layer, h, bank, dout), args.steps, args.warmup,
                                      roofline_entry="moc_xattn_bwd_dkv")
    ntok = cfg["B"] * cfg["L"]
    fl = algorithmic_flops(cfg, n_unique)
    tflops = fl["step"] / (ms * 1e-3) / 1e12

    flop_key = {"moc_kv_project": "kv_project_launch", "moc_xattn_fwd": "xattn_fwd_launch",
                "moc_xattn_bwd_dq": "xattn_bwd_dq_launch", "moc_xattn_bwd_dkv": "xattn_bwd_dkv_launch",
                "moc_chapter_project": "kv_project_launch", "moc_chapter_wgrad": "kv_project_launch",
                "moc_chapter_dx": "kv_project_launch", "moc_rows_linear:q_proj": "q", "moc_rows_linear:o_proj": "o",
                "moc_rows_linear:o_proj_dx": "o", "moc_rows_linear:q_proj_dx": "q", "moc_linear_wgrad:o_proj": "o",
                "moc_linear_wgrad:q_proj": "q"}
    roofline = None
    if dom in flop_key and live:
        ach = fl[flop_key[dom]] / (live["avg_ms"] * 1e-3) / 1e12
        roofline = {"kernel": dom, "bound": "mfma", "achieved": round(ach, 2), "peak": MFMA_BF16_PEAK_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(ach / MFMA_BF16_PEAK_TFLOPS, 4),
                    **traffic_fields("c3", dom), **counter_fields("c3", dom),
                    "avg_ms": round(live["avg_ms"], 4), "algorithmic_flop": fl[flop_key[dom]]}
    kernels = {}
    for n, v in sorted(per_kernel.items(), key=lambda kv: -kv[1]["ms_per_step"]):
        e = {"avg_ms": round(v["avg_ms"], 4), "calls": v["calls_per_step"]}
        if n in SIDE_STREAM_STAGES:
            # runs beside the main stream's kernels: its event span includes time shared with
            # them, so it is no kernel duration and gets no rate
            e["stream"] = "side (overlapped)"
        elif n in flop_key:
            e["tflops"] = round(fl[flop_key[n]] / (v["avg_ms"] * 1e-3) / 1e12, 1)
        kernels[n] = e

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(cfg, args.cpu_budget)

    # the other GPU workloads of BASELINE, timed in the same run (their own lines via --workload)
    others = {}
    if not args.headline_only:
        del layer, h, bank, dout
        torch.cuda.empty_cache()
        for name, fn in (("c5", run_c5), ("c4", lambda a: run_c4(a, losses_timing=False))):
            sub = fn(args)
            others[name] = {k: sub[k] for k in ("metric", "value", "unit", "ms_per_step", "config", "roofline")
                            if k in sub}
            for k in ("graph_replay", "hbm_frac", "tflops", "mfma_frac"):
                if k in sub:
                    others[name][k] = sub[k]
            torch.cuda.empty_cache()

    line = {
        "metric": "memory-xattn fwd+bwd tokens/s & %MFMA peak (L=1024,d=768,k=64,T=64)",
        "value": round(ntok / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) hidden states, N(0,0.02) bank and weights, random-init)",
        "config": {"workload": "c3: paper-shape sequence-routed memory layer fwd+bwd", "B": cfg["B"],
                   "L": cfg["L"], "d": cfg["d"], "heads": cfg["H"], "kv_heads": cfg["HK"],
                   "bank_tokens": cfg["C"] * cfg["T"], "chapters": cfg["C"], "tokens_per_chapter": cfg["T"],
                   "shared_chapters": cfg["S"], "top_k": cfg["k"], "routed_scale": cfg["scale"],
                   "unique_chapters": n_unique},
        "tflops": round(tflops, 2),
        "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
        "algorithmic_gflop_per_step": round(fl["step"] / 1e9, 1),
        "roofline": roofline,
        "kernels": kernels,
        "cpu_baseline": cpu,
        **others,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
