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

    ncores = min(16, len(os.sched_getaffinity(0)))
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
            "sample": f"oracle sequence_memory_layer fwd+bwd fp32, 1 sequence x {L} tokens at the full paper shape "
                      f"(d={d}, H={H}, bank {C * T} rows, k={k}); median of {iters} iterations "
                      f"({med * 1e3:.0f} ms each)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); "
              "the path shards by sequence with no exchange in the forward, see DESIGN.md", file=sys.stderr)
        sys.exit(2)

    import torch
    from memory_amd import _lib

    dev = torch.device("cuda", 0)
    dtype = torch.bfloat16
    cfg = dict(CFG)
    layer, h, bank, dout = build_inputs(dev, dtype, cfg)
    for _ in range(args.warmup):
        run_step(layer, h, bank, dout)
    torch.cuda.synchronize()

    # unique chapters of this batch (for the per-launch FLOP count of the projection)
    with torch.no_grad():
        idx_star, _, _ = layer.route(h, return_losses=False)
        n_unique = int(torch.unique(idx_star).numel())

    _lib.KERNEL_EVENTS = {}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run_step(layer, h, bank, dout)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    events = _lib.KERNEL_EVENTS
    _lib.KERNEL_EVENTS = None

    ms = wall * 1e3 / args.steps
    ntok = cfg["B"] * cfg["L"]
    fl = algorithmic_flops(cfg, n_unique)
    tflops = fl["step"] / (ms * 1e-3) / 1e12

    per_kernel = {}
    for name, pairs in events.items():
        durs = [a.elapsed_time(b) for a, b in pairs]
        per_kernel[name] = {"calls_per_step": len(pairs) / args.steps, "avg_ms": sum(durs) / len(durs),
                            "ms_per_step": sum(durs) / args.steps}
    dom = max(per_kernel, key=lambda n: per_kernel[n]["ms_per_step"])
    flop_key = {"moc_kv_project": "kv_project_launch", "moc_xattn_fwd": "xattn_fwd_launch",
                "moc_xattn_bwd_dq": "xattn_bwd_dq_launch", "moc_xattn_bwd_dkv": "xattn_bwd_dkv_launch"}
    roofline = None
    if dom in flop_key:
        ach = fl[flop_key[dom]] / (per_kernel[dom]["avg_ms"] * 1e-3) / 1e12
        roofline = {"kernel": dom, "bound": "mfma", "achieved": round(ach, 2), "peak": MFMA_BF16_PEAK_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(ach / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None,
                    "avg_ms": round(per_kernel[dom]["avg_ms"], 4), "algorithmic_flop": fl[flop_key[dom]]}
    kernels = {}
    for n, v in sorted(per_kernel.items(), key=lambda kv: -kv[1]["ms_per_step"]):
        e = {"avg_ms": round(v["avg_ms"], 4), "calls": v["calls_per_step"]}
        if n in flop_key:
            e["tflops"] = round(fl[flop_key[n]] / (v["avg_ms"] * 1e-3) / 1e12, 1)
        kernels[n] = e

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(cfg, args.cpu_budget)

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
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
