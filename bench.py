"""Benchmark of the north-star workload on one MI355X.

Workload: quant_only K3V2 over a full
Llama-3-70B-shaped cache, 80 layers x K,V bf16 [1, 8, 131072, 128] (40 GiB),
synthetic keys N(0,1) with 4 outlier channels per head x8 then RoPE (base
5e5), values N(0, 0.5^2).  One step is the drop-in compress of the whole
cache: one fused-quantizer launch over the 80 key tensors and one over the 80
value tensors, each writing fp16 reconstructions plus packed codes.

    python bench.py [--steps K] [--warmup W] [--no-cpu-baseline]

Prints one JSON line.  value = GB/s of fp16 KV compressed (2 bytes x elements
/ step time); roofline = the key-launch kernel's algorithmic bytes / its mean
HIP-event duration against 8 TB/s; cpu_baseline = the Tier-A torch oracle on
the host, on layers {0, 40, 79} (a bounded sample), scaled to the same unit.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "GB/s fp16 KV compressed (quant_only K3V2, 70B-shape 128K ctx); % HBM roofline"
HBM_PEAK_GBS = 8000.0
LAYERS, HEADS, SEQ, DIM = 80, 8, 131072, 128
BASE = 500000.0


def synth_layer(gen, device, torch):
    """One layer of keys/values with the BASELINE distribution (bf16)."""
    from nexusquant_amd.rope import device_table
    kp = torch.randn(1, HEADS, SEQ, DIM, device=device, generator=gen)
    idx = torch.argsort(torch.rand(HEADS, DIM, device=device, generator=gen), dim=1)[:, :4]
    scale = torch.ones(HEADS, DIM, device=device)
    scale.scatter_(1, idx, 8.0)
    kp *= scale[None, :, None, :]
    cos, sin = device_table(SEQ, DIM, BASE, None, device)
    c, s = cos[:SEQ], sin[:SEQ]
    lo, hi = kp[..., :DIM // 2], kp[..., DIM // 2:]
    k = torch.cat([lo * c - hi * s, lo * s + hi * c], dim=-1).to(torch.bfloat16)
    v = (torch.randn(1, HEADS, SEQ, DIM, device=device, generator=gen) * 0.5).to(torch.bfloat16)
    return k, v


def algorithmic_bytes(levels, is_key, n_tensors):
    """Bytes each launch must move: read bf16, write fp16 recon + syms + cosets + scales."""
    rows = HEADS * SEQ
    bits = {2: 2, 4: 3, 8: 4, 16: 5}[levels]
    per_row = DIM * 2 + DIM * 2 + DIM // 8 * bits + DIM // 64 + 4
    table = SEQ * DIM // 2 * 4 * 2 if is_key else 0
    return n_tensors * rows * per_row + table


def cpu_baseline(keys, values, torch):
    """Tier-A oracle (op-for-op torch restatement of the reference) on sampled layers."""
    from oracle import torch_ref as T
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    sample = [0, LAYERS // 2, LAYERS - 1]

    class Cache:
        pass

    elems = 0
    t_total = 0.0
    for li in sample:
        c = Cache()
        c.key_cache = [keys[li].cpu()]
        c.value_cache = [values[li].cpu()]
        elems += c.key_cache[0].numel() + c.value_cache[0].numel()
        t0 = time.perf_counter()
        T.quant_only_compress(c, 8, 4, rope_base=BASE)
        t_total += time.perf_counter() - t0
        del c
    gbs = 2.0 * elems / t_total / 1e9
    return {"value": round(gbs, 4), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"layers {sample} of {LAYERS} at the full {SEQ} tokens (K+V, {elems} elements, "
                      f"{t_total:.1f} s); Tier-A torch restatement of the reference, same inputs"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the compression path is data-parallel per layer "
              "and head, and this build runs on single-GPU boxes (see DESIGN.md, sharding).",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from nexusquant_amd import ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev).manual_seed(2)
    keys, values = [], []
    for _ in range(LAYERS):
        k, v = synth_layer(gen, dev, torch)
        keys.append(k)
        values.append(v)
    torch.cuda.synchronize()
    print(f"# inputs ready: {LAYERS} layers, {2 * LAYERS * HEADS * SEQ * DIM * 2 / 2**30:.1f} GiB bf16",
          file=sys.stderr, flush=True)

    def step(events=None):
        ek = None if events is None else (events[0], events[1])
        ev = None if events is None else (events[2], events[3])
        rk, ck = ops.quantize_tensors(keys, is_key=True, levels=8, rope_base=BASE, codes=True,
                                      launch_events=ek)
        rv, cv = ops.quantize_tensors(values, is_key=False, levels=4, codes=True,
                                      launch_events=ev)
        return rk, ck, rv, cv

    for _ in range(args.warmup):
        out = step()
        del out
    torch.cuda.synchronize()

    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        out = step(ev[i])
        del out
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall / args.steps * 1e3
    k_ms = sum(e[0].elapsed_time(e[1]) for e in ev) / args.steps
    v_ms = sum(e[2].elapsed_time(e[3]) for e in ev) / args.steps

    elements = 2 * LAYERS * HEADS * SEQ * DIM
    value = 2.0 * elements / (ms_step * 1e-3) / 1e9
    kb = algorithmic_bytes(8, True, LAYERS)
    vb = algorithmic_bytes(4, False, LAYERS)
    k_gbs = kb / (k_ms * 1e-3) / 1e9
    v_gbs = vb / (v_ms * 1e-3) / 1e9
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "quant_c2_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("key_launch_bytes")

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "quant_only K3V2 full cache, Llama-3-70B shape: 80 layers x K,V bf16 "
                        "[1, 8, 131072, 128], RoPE base 5e5; drop-in fp16 reconstruction + packed codes",
            "layers": LAYERS, "kv_heads": HEADS, "seq_len": SEQ, "head_dim": DIM,
            "key_bits": 3, "value_bits": 2, "input_dtype": "bf16",
        },
        "tokens_per_s": round(SEQ / (ms_step * 1e-3), 1),
        "roofline": {
            "bound": "hbm",
            "achieved": round(k_gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(k_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": "quant_rows_kernel<128, 8, key, bf16> (80 key tensors per launch)",
            "algorithmic_bytes_per_launch": kb,
            "launch_ms": round(k_ms, 4),
            "value_launch": {"achieved": round(v_gbs, 2), "frac": round(v_gbs / HBM_PEAK_GBS, 4),
                             "algorithmic_bytes_per_launch": vb, "launch_ms": round(v_ms, 4)},
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(keys, values, torch)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
