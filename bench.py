#!/usr/bin/env python3
"""Benchmark of the routed-expert MoE layer on one MI355X.

Workload of the reported value: decode of one token through a 3-bit top-8 MoE layer
(hidden 2048, 256 experts, intermediate 512, group 64, fp16 scale/bias), over a stack of
distinct seeded layers (>= 2.8 GB of expert weights, well beyond the 256 MB MALL) run
back to back; a step is one layer call.  Reported beside it: decode at 4 and 8 tokens,
the top-4 "fast mode", and 3-bit prefill of 512/2048/4096 Zipf-routed tokens.

`value` = achieved algorithmic HBM bandwidth of the layer at 1 token, in GB/s:
bytes_alg = U*expert_bytes + T*H*2 (x) + T*E*4 (logits) + T*H*2 (out) + T*K*8 (routing),
U = distinct experts selected, divided by the measured time per layer.

The CPU baseline is the oracle's C restatement of the reference expert MLP (K experts of a
token fanned out over threads, as the reference does) timed on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

METRIC = "MoE-layer decode µs/token + HBM GB/s; prefill tokens/s (3-bit, top-8)"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=800, help="timed layer calls (decode)")
    p.add_argument("--warmup", type=int, default=40)
    p.add_argument("--layers", type=int, default=8, help="distinct layers in the decode stack")
    p.add_argument("--prefill-steps", type=int, default=20)
    p.add_argument("--decode", default="1:8,4:8,8:8,1:4,4:4,8:4",
                   help="decode cases tokens:top_k, comma separated ('' for none)")
    p.add_argument("--prefill", default="512,2048,4096", help="prefill token counts ('' for none)")
    p.add_argument("--modes", default="graph,eager", help="decode launch modes")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    return p.parse_args()


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1)",
              file=sys.stderr)
        return 2
    import torch

    from kandiga_amd import synth
    from kandiga_amd.moe import QuantizedExperts, SparseMoeBlock

    dev = torch.device("cuda:0")
    shape = synth.SHAPES["h2048-e256-i512-k8-3bit"]
    H, E, K = shape.hidden, shape.num_experts, shape.top_k
    log(f"generating {args.layers} layers of {shape.name} ({shape.expert_bytes * E / 2**20:.0f} MiB each)")
    layers = [synth.make_layer_torch(shape, 7000 + i, dev) for i in range(args.layers)]
    experts = {k: [QuantizedExperts.from_stacked(shape.with_top_k(k), L, dev) for L in layers] for k in (8, 4)}
    log("layers resident")
    torch.cuda.synchronize()

    def bytes_alg(T, k, idx):
        U = int(torch.unique(idx).numel())
        return U * shape.expert_bytes + T * H * 2 + T * E * 4 + T * H * 2 + T * k * 8, U

    def time_decode(T, k, steps, warmup, graph):
        blocks = [SparseMoeBlock(ex) for ex in experts[k]]
        for ex in experts[k]:
            ex.reserve(T)
        ins = [synth.make_inputs_torch(shape, T, 9000 + 31 * i + T, dev) for i in range(len(blocks))]
        outs = [None] * len(blocks)
        ba, us_ = 0.0, 0.0
        for i, (b, (x, lg)) in enumerate(zip(blocks, ins)):
            _o, idx, _w = b(x, lg, return_routing=True)
            bb, U = bytes_alg(T, k, idx)
            ba += bb
            us_ += U
        ba /= len(blocks)
        us_ /= len(blocks)
        L = len(blocks)
        reps = max(1, steps // L)
        if graph:
            g = torch.cuda.CUDAGraph()
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                for i, b in enumerate(blocks):
                    outs[i] = b(*ins[i])
            torch.cuda.current_stream().wait_stream(s)
            with torch.cuda.graph(g):
                for i, b in enumerate(blocks):
                    outs[i] = b(*ins[i])

            def run():
                g.replay()
        else:
            def run():
                for i, b in enumerate(blocks):
                    outs[i] = b(*ins[i])
        for _ in range(max(1, warmup // L)):
            run()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            run()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * L)
        return dict(T=T, k=k, us_per_layer=us, gbs=ba / (us * 1e-6) / 1e9, bytes_alg=ba, unique_experts=us_,
                    calls=reps * L)

    results = {}
    cases = [tuple(int(v) for v in c.split(":")) for c in args.decode.split(",") if c]
    modes = [m for m in args.modes.split(",") if m]
    for T, k in cases:
        for graph in [m == "graph" for m in modes]:
            r = time_decode(T, k, args.steps, args.warmup, graph)
            key = f"decode_T{T}_K{k}_{'graph' if graph else 'eager'}"
            results[key] = r
            log(f"{key}: {r['us_per_layer']:.2f} us/layer  {r['gbs']:.0f} GB/s  U={r['unique_experts']:.1f}")

    prefill = {}
    ptoks = [int(v) for v in args.prefill.split(",") if v]
    if ptoks:
        ex = experts[8][0]
        blk = SparseMoeBlock(ex)
        for T in ptoks:
            x, lg = synth.make_inputs_torch(shape, T, 12000 + T, dev, zipf=True)
            ex.reserve(T)
            for _ in range(3):
                blk(x, lg)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(args.prefill_steps):
                blk(x, lg)
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / args.prefill_steps
            flops = 2.0 * T * K * 3 * H * shape.intermediate
            prefill[f"prefill_T{T}"] = dict(T=T, us=us, tokens_per_s=T / (us * 1e-6), tflops=flops / (us * 1e-6) / 1e12,
                                            mfma_frac=flops / (us * 1e-6) / 1e12 / MFMA_F16_PEAK_TFLOPS)
            log(f"prefill T={T}: {us:.1f} us  {T / (us * 1e-6) / 1e6:.2f} M tok/s  "
                f"{flops / (us * 1e-6) / 1e12:.1f} TFLOP/s")

    head = results.get("decode_T1_K8_graph") or next(iter(results.values()), None)
    if head is None:
        print(json.dumps({"metric": METRIC, "detail": prefill}), flush=True)
        return 0
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(layers[0], shape, args.cpu_seconds)

    line = {
        "metric": METRIC,
        "value": round(head["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": head["calls"],
        "warmup": args.warmup,
        "ms_per_step": round(head["us_per_layer"] / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u3 codes, fp16 activations, fp32 accumulate",
        "data": "synthetic (seeded MLX-layout 3-bit experts, fp16 scale/bias; random-init)",
        "config": {"workload": "moe-layer decode, 1 token, 3-bit top-8, hidden 2048, 256 experts, "
                               "intermediate 512, group 64; stack of %d distinct layers" % args.layers,
                   "tokens": 1, "top_k": K, "hidden": H, "experts": E, "intermediate": shape.intermediate,
                   "bits": 3, "layers_rotated": args.layers},
        "decode_us_per_token_layer": round(head["us_per_layer"], 3),
        "roofline": {"bound": "hbm", "achieved": round(head["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["gbs"] / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "whole layer (all kernels of one call), per-call time"},
        "cpu_baseline": cpu,
        "detail": {**{k: {kk: (round(vv, 3) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                      for k, v in results.items()},
                   **{k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                      for k, v in prefill.items()}},
    }
    print(json.dumps(line), flush=True)
    return 0


def cpu_baseline(layer_t, shape, seconds):
    """Oracle C restatement of the reference expert MLP on this host's cores (T=1, K=8)."""
    import numpy as np
    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import moe_oracle as O
    from kandiga_amd import synth

    threads = min(shape.top_k, os.cpu_count() or 1, 16)
    ntok = 64
    x, logits = synth.make_inputs(shape, ntok, 424242)
    idx, w = O.route(logits, shape.top_k)
    uniq, inv = np.unique(idx, return_inverse=True)
    ex = torch.as_tensor(uniq.astype(np.int64), device=layer_t["gate_w"].device)
    sub = {}
    for k, v in layer_t.items():
        a = v.index_select(0, ex).cpu().numpy()
        sub[k] = a.view(np.uint32) if k.endswith("_w") else a.view(np.uint16)
    pos = inv.reshape(idx.shape).astype(np.int32)
    log(f"cpu baseline: oracle expert MLP, {threads} threads, up to {seconds:.0f} s")
    O.switch_mlp(sub, x[:1], pos[:1], shape.bits, nthreads=threads)  # warm
    t0 = time.perf_counter()
    n = 0
    while n < ntok and (time.perf_counter() - t0) < seconds:
        O.switch_mlp(sub, x[n:n + 1], pos[n:n + 1], shape.bits, nthreads=threads)
        n += 1
    dt = (time.perf_counter() - t0) / n
    ba = shape.top_k * shape.expert_bytes + shape.hidden * 4 + shape.num_experts * 4 + shape.top_k * 8
    return {"value": round(ba / dt / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{n} decode tokens (1 token x top-8 experts each) of the hidden-2048 3-bit layer, "
                      f"weights resident in RAM; {dt * 1e3:.2f} ms/token",
            "us_per_token": round(dt * 1e6, 1)}


if __name__ == "__main__":
    sys.exit(main())
