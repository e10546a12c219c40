#!/usr/bin/env python3
"""Benchmark of the routed-expert MoE layer on one MI355X.

Workload of the reported value: decode of one token through a 3-bit top-8 MoE layer
(hidden 2048, 256 experts, intermediate 512, group 64, fp16 scale/bias), over a stack of 8
distinct seeded layers (2.8 GB of expert weights resident).  Each layer is called with P
different token inputs in turn, P chosen so that one pass over the call sequence touches at
least 1 GiB of distinct expert bytes (over 4x the 256 MB memory-side cache), so the bytes come
from HBM.  A step is one layer call; exactly --steps calls are timed (whole replays of the
captured sequence plus one captured partial sequence for the remainder).  Beside it: the
spread over at least 5 replays (at least 200 calls), decode at 4 and 8 tokens, the top-4 "fast
mode", 4-bit decode (the 4-bit layer of the reference's CPU path), 3-bit prefill of
512/2048/4096 Zipf-routed tokens, the hidden-2560 layer with its dense shared expert, the
hidden-4096 / 512-expert / top-10 layer's 4096-token prefill, one decode token through a
stack of 60 such layers (169 GB resident), the whole MoE block (router projection, routed
experts, gated shared expert, residual) at 1 and 8 tokens, and the TQ3 expert MLP at 1 and 4
tokens.

`value` = achieved algorithmic HBM bandwidth of the layer at 1 token, in GB/s (with --decode
lists that leave out 1:8, of the first case measured; `config` then names that case):
bytes_alg = U*expert_bytes + T*H*2 (x) + T*E*4 (logits) + T*H*2 (out) + T*K*8 (routing),
U = distinct experts selected, divided by the measured time per layer call.

`roofline` is that of the dominant kernel of the decode call (the one with the largest share of
its time), timed with HIP events around each of its launches (kmoe_profile_begin/end) in an
eager pass over the same calls, with the algorithmic bytes per launch of that kernel.
`traffic` comes from the rocprofv3 FETCH_SIZE / WRITE_SIZE summary committed under profiles/
for that kernel and workload (null when absent).

The CPU baseline restates the reference's portable scalar expert MLP (its non-NEON loops, at
the reference build's -O2 with the host's instruction set; oracle/ref_scalar.c), the K experts
of a token spread over an OpenMP team as the reference spreads them over GCD, timed on this
host: the 3-bit decode layer and the 4-bit one.  The oracle's own C restatement (the
checker: NEON accumulation order, no contraction) is reported beside it.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

METRIC = "MoE-layer decode µs/token + HBM GB/s; prefill tokens/s (3-bit, top-8)"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
ROTATE_BYTES = 1.05 * 2 ** 30  # distinct expert bytes touched per pass over the decode sequence
HERE = os.path.dirname(os.path.abspath(__file__))
PROFILES = os.path.join(HERE, "profiles")


def traffic_file(kernel: str) -> str:
    """Counter summary of `kernel` at the headline workload (decode, 1 token, top-8)."""
    return os.path.join(PROFILES, f"{kernel}_decode_t1_k8_traffic.json")


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=800, help="timed layer calls per decode case")
    p.add_argument("--warmup", type=int, default=40)
    p.add_argument("--layers", type=int, default=8, help="distinct layers in the decode stack")
    p.add_argument("--prefill-steps", type=int, default=20)
    p.add_argument("--decode", default="1:8,4:8,8:8,1:4,4:4,8:4",
                   help="decode cases tokens:top_k, comma separated ('' for none)")
    p.add_argument("--prefill", default="512,2048,4096", help="prefill token counts ('' for none)")
    p.add_argument("--modes", default="graph,eager", help="decode launch modes")
    p.add_argument("--no-prefill-copy", dest="prefill_copy", action="store_false",
                   help="skip the prefill runs that read the weights from a prefill copy")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--no-shared-layer", dest="shared_layer", action="store_false",
                   help="skip the hidden-2560 layer with the dense shared expert")
    p.add_argument("--no-wide-prefill", dest="wide_prefill", action="store_false",
                   help="skip the 4096-token prefill of the hidden-4096 / 512-expert layer")
    p.add_argument("--no-stack60", dest="stack60", action="store_false",
                   help="skip the 60-layer hidden-4096 / 512-expert / top-10 decode stack (~169 GB resident)")
    p.add_argument("--x-dtype", default="f16", choices=("f16", "bf16", "f32"),
                   help="activation dtype of the routed-layer cases (the shared-expert layer stays fp16)")
    p.add_argument("--no-block", dest="block", action="store_false",
                   help="skip the whole-block decode (router, routed experts, gated shared expert, residual)")
    p.add_argument("--no-tq3", dest="tq3", action="store_false",
                   help="skip the TQ3 codebook expert MLP at 1 and 4 tokens")
    p.add_argument("--no-4bit", dest="four_bit", action="store_false",
                   help="skip the 4-bit decode layer (GPU and CPU)")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only run 5 device copies of 256 MiB (the known-size kernel that the "
                        "FETCH_SIZE / WRITE_SIZE counters are calibrated against) and exit")
    return p.parse_args()


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1)",
              file=sys.stderr)
        return 2
    import torch

    if args.copy_calibration:
        a = torch.ones(256 * 2 ** 20, dtype=torch.uint8, device="cuda:0")
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": a.numel(), "copies": 5}), flush=True)
        return 0

    from kandiga_amd import synth
    from kandiga_amd.moe import QuantizedExperts, SparseMoeBlock, profile_kernels

    X_DTYPES = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}
    XB = {"f16": 2, "bf16": 2, "f32": 4}[args.x_dtype]  # bytes per activation element

    dev = torch.device("cuda:0")
    shape = synth.SHAPES["h2048-e256-i512-k8-3bit"]
    H, E, I = shape.hidden, shape.num_experts, shape.intermediate
    log(f"generating {args.layers} layers of {shape.name} ({shape.expert_bytes * E / 2**20:.0f} MiB each)")
    layers = [synth.make_layer_torch(shape, 7000 + i, dev) for i in range(args.layers)]
    experts = {k: [QuantizedExperts.from_stacked(shape.with_top_k(k), L, dev) for L in layers] for k in (8, 4)}
    del layers
    torch.cuda.synchronize()
    log("layers resident")
    copy_gbs = measured_copy_gbs(torch, dev)
    log(f"device copy: {copy_gbs:.0f} GB/s (read + write)")

    def kernel_bytes(name, shp, T, k, U):
        """Algorithmic bytes of one launch of a decode-path kernel."""
        H, E, I = shp.hidden, shp.num_experts, shp.intermediate
        gu = 2 * I * H * shp.bits // 8 + 4 * I * (H // 64) * 2
        dn = H * I * shp.bits // 8 + 2 * H * (I // 64) * 2
        act = T * k * I * 4
        if name == "dec_stage1_kernel":
            return U * gu + T * H * XB + T * E * 4 + act + T * k * 8
        if name == "dec_stage2_kernel":
            return U * dn + act + T * H * 2 + T * k * 8
        return U * shp.expert_bytes + T * H * XB + T * E * 4 + T * H * 2 + T * k * 8

    def decode_case(T, k, graph, exs=None, shp=None, profile=True, steps=None):
        exs = exs if exs is not None else experts[k]
        shp = shp or shape
        steps = args.steps if steps is None else steps
        H, E, I = shp.hidden, shp.num_experts, shp.intermediate
        blocks = [SparseMoeBlock(ex) for ex in exs]
        for ex in exs:
            ex.reserve(T)
        # Input sets are added until one pass over the sequence touches ROTATE_BYTES of distinct
        # expert weights (counted from the routing itself): every layer with input set 0, then 1, ...
        seq, uniq, seen = [], [], [set() for _ in blocks]
        p = 0
        while p < 64:
            for li, b in enumerate(blocks):
                x, lg = synth.make_inputs_torch(shp, T, 9000 + 997 * p + 31 * li + T, dev)
                if not shp.shared_intermediate:  # the dense shared expert takes fp16 x only
                    x = x.to(X_DTYPES[args.x_dtype])
                _o, idx, _w = b(x, lg, return_routing=True)
                ids = torch.unique(idx).tolist()
                seen[li].update(ids)
                uniq.append(len(ids))
                seq.append((li, b, x, lg))
            p += 1
            if sum(len(q) for q in seen) * shp.expert_bytes >= ROTATE_BYTES:
                break
        P = p
        n = len(seq)
        distinct = sum(len(q) for q in seen) * shp.expert_bytes
        xb = 2 if shp.shared_intermediate else XB
        b_alg = [U * shp.expert_bytes + shp.shared_bytes + T * H * xb + T * E * 4 + T * H * 2 + T * k * 8
                 for U in uniq]
        outs = [None] * n
        if graph:
            def capture(calls):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    for i, (_li, b, x, lg) in enumerate(calls):
                        outs[i] = b(x, lg)
                return g
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                for _li, b, x, lg in seq:
                    b(x, lg)
            torch.cuda.current_stream().wait_stream(s)
            g_full = capture(seq)
            r = steps % n
            g_rem = capture(seq[:r]) if r else None

            def run_full():
                g_full.replay()

            def run_steps():
                for _ in range(steps // n):
                    g_full.replay()
                if g_rem is not None:
                    g_rem.replay()
        else:
            def run_full():
                for i, (_li, b, x, lg) in enumerate(seq):
                    outs[i] = b(x, lg)

            def run_steps():
                for j in range(steps):
                    _li, b, x, lg = seq[j % n]
                    b(x, lg)
        for _ in range(max(1, math.ceil(args.warmup / n))):
            run_full()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        run_steps()          # exactly `steps` layer calls
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / steps
        # bytes of the timed calls: full passes plus the first `steps % n` calls
        timed_bytes = (steps // n) * sum(b_alg) + sum(b_alg[:steps % n])
        ba = timed_bytes / steps
        r = dict(T=T, k=k, us_per_layer=us, gbs=ba / (us * 1e-6) / 1e9, bytes_alg=ba, steps=steps,
                 unique_experts=sum(uniq) / n, calls_per_replay=n, inputs_per_layer=P,
                 distinct_expert_bytes_per_replay=distinct)
        # spread: at least 5 replays and 200 calls, an event between replays (the events add a
        # little, so the exact-steps figure above stays the one reported)
        reps = max(5, math.ceil(200 / n))
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
        ev[0].record()
        for i in range(reps):
            run_full()
            ev[i + 1].record()
        torch.cuda.synchronize()
        per = sorted(ev[i].elapsed_time(ev[i + 1]) * 1e3 / n for i in range(reps))
        r["spread"] = {"replays": reps, "calls": reps * n}
        for name, f in (("us_p10", 0.1), ("us_median", 0.5), ("us_p90", 0.9)):
            r[name] = per[min(len(per) - 1, int(round(f * (len(per) - 1))))]
        if graph and profile:
            # per-kernel event timing over one eager pass of the same calls
            with profile_kernels(8 * n + 16) as prof:
                for _li, b, x, lg in seq:
                    b(x, lg)
            kern = {}
            Umean = sum(uniq) / n
            for name, v in prof.result.items():
                ab = sum(kernel_bytes(name, shp, T, k, U) for U in uniq) / n
                kern[name] = {"mean_us": v["mean_ms"] * 1e3, "launches": v["launches"], "bytes_alg": ab,
                              "gbs": ab / (v["mean_ms"] * 1e-3) / 1e9}
            r["kernels"] = kern
            r["dominant_kernel"] = max(kern, key=lambda nm: kern[nm]["mean_us"]) if kern else None
            del Umean
        return r

    results = {}
    cases = [tuple(int(v) for v in c.split(":")) for c in args.decode.split(",") if c]
    modes = [m for m in args.modes.split(",") if m]
    for T, k in cases:
        for graph in [m == "graph" for m in modes]:
            r = decode_case(T, k, graph)
            key = f"decode_T{T}_K{k}_{'graph' if graph else 'eager'}"
            results[key] = r
            extra = "".join(f"  {nm} {v['mean_us']:.2f} us ({v['gbs']:.0f} GB/s)" for nm, v in r.get("kernels", {}).items())
            log(f"{key}: {r['us_per_layer']:.2f} us/layer over {r['steps']} calls (replays p10/median/p90 "
                f"{r['us_p10']:.2f}/{r['us_median']:.2f}/{r['us_p90']:.2f})  {r['gbs']:.0f} GB/s  "
                f"U={r['unique_experts']:.1f} P={r['inputs_per_layer']} "
                f"distinct={r['distinct_expert_bytes_per_replay'] / 2**30:.2f} GiB{extra}")

    def prefill_case(ex, shp, T, tag=""):
        blk = SparseMoeBlock(ex)
        H, I = shp.hidden, shp.intermediate
        x, lg = synth.make_inputs_torch(shp, T, 12000 + T, dev, zipf=True)
        if not shp.shared_intermediate:  # the dense shared expert takes fp16 x only
            x = x.to(X_DTYPES[args.x_dtype])
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
        with profile_kernels(64) as prof:
            for _ in range(3):
                blk(x, lg)
        kern = {n: round(v["mean_ms"] * 1e3, 2) for n, v in prof.result.items()}
        flops = 2.0 * T * shp.top_k * 3 * H * I + 2.0 * T * 3 * H * shp.shared_intermediate
        gemm_us = kern.get("gemm_gateup_kernel", 0) + kern.get("gemm_down_kernel", 0)
        r = dict(T=T, us=us, tokens_per_s=T / (us * 1e-6), tflops=flops / (us * 1e-6) / 1e12,
                 mfma_frac=flops / (us * 1e-6) / 1e12 / MFMA_F16_PEAK_TFLOPS, kernel_us=kern,
                 gemm_mfma_frac=(2.0 * T * shp.top_k * 3 * H * I / (gemm_us * 1e-6) / 1e12 / MFMA_F16_PEAK_TFLOPS)
                 if gemm_us else None)
        log(f"prefill{tag} T={T}: {us:.1f} us  {T / (us * 1e-6) / 1e6:.2f} M tok/s  "
            f"{flops / (us * 1e-6) / 1e12:.1f} TFLOP/s  kernels(us) {kern}")
        return r

    prefill = {}
    for T in [int(v) for v in args.prefill.split(",") if v]:
        prefill[f"prefill_T{T}"] = prefill_case(experts[8][0], shape, T)
    if args.prefill_copy and args.prefill:
        ex_pk = experts[8][0].with_prefill_copy()
        for T in [int(v) for v in args.prefill.split(",") if v]:
            prefill[f"prefill_copy_T{T}"] = prefill_case(ex_pk, shape, T, " (prefill copy)")
        del ex_pk

    # the whole MoE block (router projection, routed experts, gated shared expert, residual) on the
    # same 8 resident layers, decode over enough inputs that a replay touches >= 1 GiB of experts
    if args.block and args.decode:
        results.update(block_cases(torch, dev, shape, experts[8], args.steps, log))

    # the hidden-2560 layer with a dense fp16 shared expert (decode over 4 rotated layers)
    if args.shared_layer:
        shp4 = synth.SHAPES["h2560-e256-i1024-k8-3bit-shared1024"]
        log(f"generating 4 layers of {shp4.name}")
        ex4 = [QuantizedExperts.from_stacked(shp4, synth.make_layer_torch(shp4, 7100 + i, dev), dev)
               for i in range(4)]
        torch.cuda.synchronize()
        for T in (1, 8):
            r = decode_case(T, 8, True, ex4, shp4, profile=False)
            results[f"shared_layer_decode_T{T}_K8_graph"] = r
            log(f"{shp4.name} decode T={T}: {r['us_per_layer']:.2f} us/layer  {r['gbs']:.0f} GB/s (incl. shared "
                f"expert bytes)")
        prefill["shared_layer_prefill_T2048"] = prefill_case(ex4[0], shp4, 2048, " (hidden 2560 + shared)")
        del ex4
        torch.cuda.empty_cache()

    # the hidden-4096 / 512-expert / top-10 layer at 4096 prefill tokens
    if args.wide_prefill and args.prefill:
        shp6 = synth.SHAPES["h4096-e512-i1024-k10-3bit"]
        log(f"generating 1 layer of {shp6.name}")
        ex6 = QuantizedExperts.from_stacked(shp6, synth.make_layer_torch(shp6, 7300, dev), dev)
        torch.cuda.synchronize()
        prefill["wide_layer_prefill_T4096"] = prefill_case(ex6, shp6, 4096, " (hidden 4096, 512 experts, top-10)")
        if args.prefill_copy:
            ex6c = ex6.with_prefill_copy()
            prefill["wide_layer_prefill_copy_T4096"] = prefill_case(
                ex6c, shp6, 4096, " (hidden 4096, 512 experts, top-10, prefill copy)")
            del ex6c
        del ex6
        torch.cuda.empty_cache()

    # 60 independent hidden-4096 / 512-expert / top-10 layers resident (~169 GB): one decode
    # token through the whole stack per replay
    if args.stack60:
        shp5 = synth.SHAPES["h4096-e512-i1024-k10-3bit"]
        log(f"generating 60 layers of {shp5.name} ({shp5.expert_bytes * shp5.num_experts * 60 / 1e9:.0f} GB)")
        ex5 = [QuantizedExperts.from_stacked(shp5, synth.make_layer_torch(shp5, 7200 + i, dev), dev)
               for i in range(60)]
        torch.cuda.synchronize()
        r = decode_case(1, 10, True, ex5, shp5, profile=False, steps=max(args.steps, 60))
        r["us_per_token_60_layers"] = r["us_per_layer"] * 60
        results["stack60_decode_T1_K10_graph"] = r
        log(f"60-layer {shp5.name} stack, decode T=1: {r['us_per_layer']:.2f} us/layer, "
            f"{r['us_per_layer'] * 60:.1f} us/token, {r['gbs']:.0f} GB/s")
        del ex5
        torch.cuda.empty_cache()

    # the 4-bit layer of the reference's CPU path (hidden 2048, 256 experts, intermediate 512,
    # top-8): decode of one token on the GPU over a rotated stack, like the 3-bit headline
    shp1 = synth.SHAPES["h2048-e256-i512-k8-4bit"]
    if args.four_bit and args.decode:
        experts.clear()
        torch.cuda.empty_cache()
        log(f"generating {args.layers} layers of {shp1.name}")
        ex1 = [QuantizedExperts.from_stacked(shp1, synth.make_layer_torch(shp1, 7400 + i, dev), dev)
               for i in range(args.layers)]
        torch.cuda.synchronize()
        r = decode_case(1, 8, True, ex1, shp1, profile=False)
        results["4bit_decode_T1_K8_graph"] = r
        log(f"{shp1.name} decode T=1: {r['us_per_layer']:.2f} us/layer  {r['gbs']:.0f} GB/s")
        del ex1
        torch.cuda.empty_cache()

    # TQ3 codebook experts of the same shape (hidden 2048, 256 experts, intermediate 512, top-8):
    # the switch_mlp contract through kmoe_tq3_expert_mlp, graph-replayed over 3 layers with
    # enough token inputs that one pass touches over 1 GiB of distinct expert bytes
    if args.tq3 and args.decode:
        experts.clear()
        torch.cuda.empty_cache()
        results.update(tq3_cases(torch, dev, shape, args.steps, profile_kernels, log))

    head = results.get("decode_T1_K8_graph") or next(iter(results.values()), None)
    if head is None:
        print(json.dumps({"metric": METRIC, "detail": prefill}), flush=True)
        return 0
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(shape, args.cpu_seconds, shp1 if args.four_bit else None)

    roof = {"bound": "hbm", "achieved": None, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": None, "traffic": None}
    dk = head.get("dominant_kernel")
    if dk:
        kv = head["kernels"][dk]
        roof.update(achieved=round(kv["gbs"], 1), frac=round(kv["gbs"] / HBM_PEAK_GBS, 4), kernel=dk,
                    mean_launch_us=round(kv["mean_us"], 3), bytes_alg_per_launch=round(kv["bytes_alg"]),
                    frac_of_measured_copy=round(kv["gbs"] / copy_gbs, 4))
        # the committed counter summaries cover the 1-token top-8 workload only
        if head["T"] == 1 and head["k"] == 8:
            roof["traffic"] = kernel_traffic(dk)

    line = {
        "metric": METRIC,
        "value": round(head["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": head["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(head["us_per_layer"] / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u3",
        "data": "synthetic (seeded MLX-layout 3-bit experts, fp16 scale/bias, %s activations; random-init)"
                % {"f16": "fp16", "bf16": "bf16", "f32": "fp32"}[args.x_dtype],
        "config": {"workload": "moe-layer decode, %d token%s, 3-bit top-%d, hidden 2048, 256 experts, "
                               "intermediate 512, group 64; stack of %d distinct layers, %d inputs per layer"
                               % (head["T"], "" if head["T"] == 1 else "s", head["k"], args.layers,
                                  head["inputs_per_layer"]),
                   "tokens": head["T"], "top_k": head["k"], "hidden": H, "experts": E, "intermediate": I,
                   "bits": 3, "layers_rotated": args.layers},
        "decode_us_per_token_layer": round(head["us_per_layer"] / head["T"], 3),
        "roofline": roof,
        "cpu_baseline": cpu,
        "detail": {"measured_copy_GBs": round(copy_gbs, 1),
                   **{k: {kk: (round(vv, 3) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                      for k, v in results.items()},
                   **{k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                      for k, v in prefill.items()}},
    }
    print(json.dumps(line), flush=True)
    return 0


def block_cases(torch, dev, shape, layers, steps, log) -> dict:
    """The whole MoE block of a Qwen-style layer (kmoe_block_forward) at 1 and 8 tokens: a 4-bit
    bf16-scale router projection [256, 2048] and shared expert (intermediate 512, sigmoid gate)
    around each of the resident 3-bit routed layers, a residual, fp16 out.  Graph replay over
    enough token inputs per layer that a replay touches >= 1 GiB of distinct routed experts;
    GB/s counts the distinct routed experts, the router, shared expert and gate bytes, x,
    residual and out."""
    from kandiga_amd import synth
    from kandiga_amd.moe import MoEBlock

    H, E, K, Is = shape.hidden, shape.num_experts, shape.top_k, 512
    blocks = [MoEBlock.from_arrays(ex, synth.make_block(shape, Is, 8300 + i, bits=4, scale_dtype="bf16"), 4, "bf16")
              for i, ex in enumerate(layers)]
    q4 = lambda rows, cols: rows * cols // 2 + 2 * rows * (cols // 64) * 2  # 4-bit codes + bf16 s, b
    extra = q4(E, H) + 2 * q4(Is, H) + q4(H, Is) + q4(1, H)
    out = {}
    g = torch.Generator(device=dev)
    g.manual_seed(8400)
    for T in (1, 8):
        seq, seen, uniq = [], [set() for _ in blocks], []
        p = 0
        while p < 64:
            for li, b in enumerate(blocks):
                b.workspace(T)
                x = torch.randn((T, H), device=dev, generator=g).half()
                res = torch.randn((T, H), device=dev, generator=g).half()
                _o, idx, _w, _lg = b(x, res, return_routing=True)
                ids = torch.unique(idx).tolist()
                seen[li].update(ids)
                uniq.append(len(ids))
                seq.append((b, x, res))
            p += 1
            if sum(len(q) for q in seen) * shape.expert_bytes >= 2 ** 30:
                break
        n = len(seq)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for b, x, res in seq:
                b(x, res)
        reps = max(5, -(-steps // n))
        gr.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            gr.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * n)
        U = sum(uniq) / n
        ba = U * shape.expert_bytes + extra + 3 * T * H * 2
        out[f"block_decode_T{T}_K{K}_graph"] = {"T": T, "k": K, "us_per_layer": us, "gbs": ba / (us * 1e-6) / 1e9,
                                                "bytes_alg": ba, "unique_experts": U, "calls": reps * n,
                                                "inputs_per_layer": p, "shared_intermediate": Is}
        log(f"MoE block decode T={T}: {us:.2f} us/layer  {ba / (us * 1e-6) / 1e9:.0f} GB/s  U={U:.1f} P={p}")
    del blocks
    return out


def tq3_cases(torch, dev, shape, steps, profile_kernels, log) -> dict:
    """The TQ3 expert MLP (switch_mlp contract, fp16 x, top-8) at 1 and 4 tokens on three seeded
    layers of 256 TQ3 experts (hidden 2048, intermediate 512; random indices, fp16 block scales
    in [0, 0.02)), captured as one graph over enough inputs per layer that a replay touches
    >= 1 GiB of distinct expert bytes.  GB/s counts the distinct experts' bytes per call plus x
    and y; per-kernel figures come from HIP events around each launch in an eager pass."""
    from kandiga_amd import tq3

    H, I, E, K = shape.hidden, shape.intermediate, shape.num_experts, 8
    eb = tq3.expert_bytes(H, I)
    g = torch.Generator(device=dev)
    g.manual_seed(8100)
    layers = []
    for _ in range(3):
        body = torch.randint(0, 256, (E, eb), dtype=torch.uint8, device=dev, generator=g)
        blk = body.view(E, -1, 20)
        for j in range(0, E, 32):  # the four fp16 block scales, in chunks to bound the temporary
            sc = (torch.rand((min(32, E - j), blk.shape[1], 4), device=dev, generator=g) * 0.02).half()
            blk[j:j + 32, :, :8] = sc.view(torch.uint8)
        layers.append(tq3.TQ3Experts(body, H, I, dev))
    out = {}
    for T in (1, 4):
        for ex in layers:
            ex.reserve(T, K)
        seq, seen, uniq = [], [set() for _ in layers], []
        p = 0
        while p < 256:
            for li, ex in enumerate(layers):
                x = (torch.randn((T, H), device=dev, generator=g) * 0.5).half()
                idx = torch.rand((T, E), device=dev, generator=g).argsort(dim=1)[:, :K].to(torch.int32).contiguous()
                ids = torch.unique(idx).tolist()
                seen[li].update(ids)
                uniq.append(len(ids))
                seq.append((ex, x, idx))
            p += 1
            if sum(len(q) for q in seen) * eb >= 2 ** 30:
                break
        n = len(seq)
        for ex, x, idx in seq:
            ex(x, idx)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for ex, x, idx in seq:
                ex(x, idx)
        reps = max(5, -(-steps // n))
        gr.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            gr.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * n)
        U = sum(uniq) / n
        ba = U * eb + T * H * 2 + T * K * H * 2
        r = {"T": T, "k": K, "us_per_call": us, "gbs": ba / (us * 1e-6) / 1e9, "bytes_alg": ba,
             "unique_experts": U, "calls": reps * n, "inputs_per_layer": p,
             "distinct_expert_bytes_per_replay": sum(len(q) for q in seen) * eb}
        with profile_kernels(4 * n + 16) as prof:
            for ex, x, idx in seq:
                ex(x, idx)
        kern = {}
        for name, v in prof.result.items():
            kern[name] = {"mean_us": v["mean_ms"] * 1e3, "launches": v["launches"]}
        launches = sorted(kern.items(), key=lambda kv: -kv[1]["mean_us"])
        r["kernels"] = kern
        out[f"tq3_T{T}_K{K}_graph"] = r
        log(f"TQ3 expert MLP T={T} K={K}: {us:.2f} us/call  {r['gbs']:.0f} GB/s  U={U:.1f} P={p}  "
            + "  ".join(f"{nm} {v['mean_us']:.2f} us x{v['launches']}" for nm, v in launches))
    del layers
    torch.cuda.empty_cache()
    return out


def measured_copy_gbs(torch, dev) -> float:
    """Read+write bandwidth of a 1 GiB device-to-device copy (a measured ceiling beside the spec)."""
    a = torch.empty(2 ** 30, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    gbs = 2 * a.numel() * 10 / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del a, b
    torch.cuda.empty_cache()
    return gbs


def kernel_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from its committed rocprofv3 counter summary:
    (FETCH_SIZE + WRITE_SIZE) KiB per dispatch, each divided by the ratio the same counter
    reads for a device copy of known size (null when there is no summary for the kernel)."""
    try:
        with open(traffic_file(kernel)) as f:
            t = json.load(f)
        fetch = t["fetch_kib_per_dispatch"] * 1024 / t["copy_fetch_ratio"]
        write = t["write_kib_per_dispatch"] * 1024 / t["copy_write_ratio"]
        return round(fetch + write)
    except (OSError, KeyError, ValueError, ZeroDivisionError):
        return None


def _cpu_time(fn, ntok, seconds):
    """Mean seconds per token of fn(i) over up to ntok tokens or `seconds` of wall time."""
    fn(0)  # warm
    t0 = time.perf_counter()
    n = 0
    while n < ntok and (time.perf_counter() - t0) < seconds:
        fn(n)
        n += 1
    return (time.perf_counter() - t0) / n, n


def cpu_baseline(shape, seconds, shape4=None):
    """The reference's portable scalar expert MLP (oracle/ref_scalar.c) on this host's cores, decode
    of one token at top-8: the 3-bit layer of the headline (its value) and, with shape4, the
    4-bit layer.  Experts are generated on the host (16 per layer: the work per token does not
    depend on which experts are picked); the oracle's checker restatement is timed beside it."""
    import numpy as np

    sys.path.insert(0, HERE)
    from oracle import moe_oracle as O
    from kandiga_amd import synth

    threads = min(shape.top_k, os.cpu_count() or 1, 16)
    ntok = 64

    def one(shp, seed, budget):
        sub_shape = synth.LayerShape(shp.hidden, shp.intermediate, 16, shp.top_k, shp.bits)
        layer = synth.make_layer(sub_shape, seed, "bf16")   # bf16 scales, as the reference stores them
        x, logits = synth.make_inputs(sub_shape, ntok, seed + 1)
        idx, _w = O.route(logits, shp.top_k)
        dt, n = _cpu_time(lambda i: O.ref_scalar_switch_mlp(layer, x[i:i + 1], idx[i:i + 1], shp.bits, "bf16",
                                                            nthreads=threads), ntok, budget)
        dt1, n1 = _cpu_time(lambda i: O.ref_scalar_switch_mlp(layer, x[i:i + 1], idx[i:i + 1], shp.bits, "bf16",
                                                              nthreads=1), ntok, budget / 4)
        dto, no = _cpu_time(lambda i: O.switch_mlp(layer, x[i:i + 1], idx[i:i + 1], shp.bits, "bf16",
                                                   nthreads=threads), ntok, budget / 4)
        ba = shp.top_k * shp.expert_bytes + shp.hidden * 4 + shp.num_experts * 4 + shp.top_k * 8
        return ba, dict(tokens=n, us_per_token=round(dt * 1e6, 1), GBs=round(ba / dt / 1e9, 3),
                        single_thread={"tokens": n1, "us_per_token": round(dt1 * 1e6, 1),
                                       "GBs": round(ba / dt1 / 1e9, 3)},
                        checker_restatement={"tokens": no, "us_per_token": round(dto * 1e6, 1),
                                             "GBs": round(ba / dto / 1e9, 3)})

    log(f"cpu baseline: reference scalar expert MLP, {threads} threads, about {seconds * 1.5:.0f} s per layer")
    ba, r3 = one(shape, 424242, seconds)
    r4 = one(shape4, 434343, seconds / 2)[1] if shape4 is not None else None
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "")
    except OSError:
        pass
    dt = r3["us_per_token"] * 1e-6
    return {"value": r3["GBs"], "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{r3['tokens']} decode tokens (1 token x top-8 experts each) of the hidden-2048 3-bit layer, "
                      f"weights resident in RAM; {dt * 1e3:.2f} ms/token; the reference's scalar loops at -O2 "
                      f"(oracle/ref_scalar.c), {threads}-thread OpenMP team",
            "us_per_token": r3["us_per_token"],
            "single_thread": r3["single_thread"],
            "checker_restatement": r3["checker_restatement"],
            "layer_4bit": r4,
            # the reference runs 3-bit prefill as one decode call per token
            "prefill_T512_s_extrapolated": round(512 * dt, 3),
            "host": {"cpu_model": model, "nproc": os.cpu_count()}}


if __name__ == "__main__":
    sys.exit(main())
