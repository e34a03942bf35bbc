"""MoE layer decode benchmark on one MI355X (BASELINE.json metric).

Workload: one DeepSeek-V3-shape MoE layer decode step with 1 token:
H=7168, 256 routed experts + 1 shared, I=2048, top-8 sigmoid routing from N(0,1) logits,
every expert EXL3 at 4 bpw (uniform random trellis, +-1 suh, +-U(0.5,1.5) svh), bf16 N(0,1)
activations. A step = routing + grouping + rotations + gate/up GEMV + SwiGLU + down GEMV +
slot reduction + shared expert (evamx_moe_forward), inputs resident in HBM.

Cache hygiene: the weights of L layer copies (257 experts each, 5.7 GB per layer at 4 bpw) stay
resident and every step uses the next layer and a fresh routing draw, so a step's 199 MB are
not served from the 256 MiB MALL. Steps are replayed from a hipGraph.

Output: one JSON line (value = achieved HBM GB/s over the algorithmic bytes of the step).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE layer decode µs + achieved HBM GB/s (DSv3 shape, 4bpw EXL3, 1/16 tok)"
PEAK_HBM = 8000.0         # GB/s, MI355X
H, I, E, TOPK = 7168, 2048, 256, 8


def proj_bytes(n_in, n_out, bits):
    return n_in * n_out * bits / 8 + 2 * (n_in + n_out)


def expert_bytes(bits, hidden=H, inter=I):
    return 2 * proj_bytes(hidden, inter, bits) + proj_bytes(inter, hidden, bits)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class DeviceLayers:
    """L layers x (E routed + 1 shared) experts, all resident, with [9, E] pointer tables."""

    def __init__(self, torch, dev, n_layers, bits, hidden=H, inter=I, n_experts=E, seed=1234):
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        self.n = n_experts + 1
        t16 = int(16 * bits)
        self.proj_elems = (hidden // 16) * (inter // 16) * t16
        nbig = n_layers * self.n * 3 * self.proj_elems
        log(f"allocating {nbig * 2 / 1e9:.1f} GB of trellis for {n_layers} layers")
        self.trellis = torch.empty(nbig, dtype=torch.int16, device=dev)
        chunk = 1 << 28
        for s in range(0, nbig, chunk):
            self.trellis[s:s + chunk].random_(-32768, 32768, generator=g)
        vec = max(hidden, inter)
        self.suh = (torch.randint(0, 2, (n_layers, self.n, 3, vec), generator=g, device=dev) * 2 - 1).half()
        mag = torch.rand((n_layers, self.n, 3, vec), generator=g, device=dev) + 0.5
        sign = torch.randint(0, 2, (n_layers, self.n, 3, vec), generator=g, device=dev) * 2 - 1
        self.svh = (mag * sign / (hidden ** 0.5)).half()
        base_t = self.trellis.data_ptr()
        base_su = self.suh.data_ptr()
        base_sv = self.svh.data_ptr()
        self.tables, self.shared = [], []
        for l in range(n_layers):
            rows = [[0] * n_experts for _ in range(9)]
            sh = [0] * 9
            for e in range(self.n):
                ptrs = []
                for p in range(3):
                    k = (l * self.n + e) * 3 + p
                    ptrs += [base_t + 2 * k * self.proj_elems, base_su + 2 * k * vec, base_sv + 2 * k * vec]
                if e < n_experts:
                    for r in range(9):
                        rows[r][e] = ptrs[r]
                else:
                    sh = ptrs
            self.tables.append(torch.tensor(rows, dtype=torch.int64, device=dev))
            self.shared.append(sh)


def cpu_baseline(seconds_hint=True):
    """PyTorch-CPU restatement on the host cores: one routed expert + the shared expert of the
    1-token layer (the sampled bytes are 2 of the 9 experts the full step reads)."""
    import numpy as np
    import torch

    from oracle import synth, torch_cpu

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    rng = np.random.default_rng(5)
    ew = [synth.expert(rng, H, I, 4, 1 / np.sqrt(H)) for _ in range(2)]
    parts = [tuple(tuple(torch.from_numpy(np.ascontiguousarray(a)) for a in ew_i.parts[p]) for p in "gud") for ew_i in ew]
    dec = torch_cpu.Decoder(4)
    x = torch.from_numpy(synth.activations_bf16(rng, 1, H))
    idx = torch.tensor([[0]])
    w = torch.tensor([[1.0]])

    def run():
        return torch_cpu.moe_layer(x, idx, w, {0: parts[0]}, parts[1], dec, 10.0)

    run()                                   # warm-up
    times = []
    while len(times) < 2 or (sum(times) < 10.0 and len(times) < 12):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t = sum(times) / len(times)
    nbytes = 2 * expert_bytes(4)
    model = ""
    try:
        model = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name"))
    except Exception:
        pass
    return {"value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"1 routed + 1 shared expert of the 1-token DSv3 layer at 4 bpw "
                      f"({nbytes / 1e6:.1f} MB; mean of {len(times)} runs after 1 warm-up; {t:.2f} s each, "
                      f"{sum(times):.1f} s timed)",
            "layer_seconds_scaled": round(t * 9 / 2, 2), "cpu_model": model,
            "torch_threads": torch.get_num_threads()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--tokens", type=int, default=1)
    ap.add_argument("--bits", type=float, default=4.0)
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--graph-steps", type=int, default=8)
    ap.add_argument("--ksplit-gu", type=int, default=0)
    ap.add_argument("--ksplit-down", type=int, default=0)
    ap.add_argument("--routing", choices=("plain", "skewed"), default=None,
                    help="N(0,1) logits, or config 3's per-token bias (default: plain at 1 token, skewed above)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 1 GiB device copy (the reference kernel for FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (see DESIGN.md, "
              "'How the path would shard'); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_calibration:
        copy_calibration(torch)
        return

    from eva_amd import ops
    from eva_amd._lib import lib

    dev = torch.device("cuda", 0)
    T = args.tokens
    if args.routing is None:
        args.routing = "plain" if T == 1 else "skewed"
    layers = DeviceLayers(torch, dev, args.layers, args.bits)
    g = torch.Generator(device=dev)
    g.manual_seed(99)
    n_draws = max(args.graph_steps, args.layers) * 2
    logits = torch.randn((n_draws, T, E), generator=g, device=dev)
    if args.routing == "skewed":
        # config 3: per-token random bias so expert loads span 0..T (2 hot experts +6 for every
        # token, 6 warm experts +3 for a per-token coin flip, a fresh draw of both per step)
        for i in range(n_draws):
            perm = torch.randperm(E, generator=g, device=dev)
            logits[i][:, perm[:2]] += 6.0
            coin = torch.randint(0, 2, (T, 6), generator=g, device=dev).float()
            logits[i][:, perm[2:8]] += 3.0 * coin
    x = torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16)
    ws = ops.MoeWorkspace(dev, rows_max=T, hidden=H, inter=I, topk=TOPK, n_local=E, has_shared=True,
                          ksplit_gu=args.ksplit_gu, ksplit_down=args.ksplit_down)
    sel = torch.empty(T, TOPK, dtype=torch.int64, device=dev)
    wts = torch.empty(T, TOPK, dtype=torch.float32, device=dev)
    out = torch.empty(T, H, dtype=torch.float32, device=dev)

    def step(i):
        l = i % args.layers
        ops.moe_forward(ws, x, layers.tables[l], out, limit=10.0, bits=args.bits, logits=logits[i % n_draws],
                        sel=sel, weights=wts, shared_ptrs=layers.shared[l], shared_bits=args.bits)

    # unique experts per step (for the algorithmic bytes), from the same routing draws
    uniq = []
    for i in range(n_draws):
        step(i)
        uniq.append(len(set(sel.reshape(-1).tolist())))
    torch.cuda.synchronize()
    if not torch.isfinite(out).all():
        raise RuntimeError("non-finite layer output")
    ebytes = expert_bytes(args.bits)
    act_bytes = T * H * 2 + T * E * 4 + T * H * 4

    G = args.graph_steps
    stream = torch.cuda.Stream(device=dev)
    graph = None
    if not args.no_graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            for i in range(G):
                step(i)
            torch.cuda.synchronize()
            with torch.cuda.graph(graph, stream=stream):
                for i in range(G):
                    step(i)
    reps = max(1, args.steps // G)
    steps = reps * G
    mean_uniq = sum(uniq[i % n_draws] for i in range(G)) / G
    step_bytes = (mean_uniq + 1) * ebytes + act_bytes

    def run_block(n):
        with torch.cuda.stream(stream):
            if graph is not None:
                for _ in range(n):
                    graph.replay()
            else:
                for i in range(n * G):
                    step(i)

    run_block(max(1, args.warmup // G))
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    run_block(reps)
    ev1.record(stream)
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1)
    us_step = ms * 1e3 / steps
    gbps = step_bytes / (us_step * 1e-6) / 1e9
    log(f"{steps} steps, {us_step:.2f} us/step, {gbps:.1f} GB/s (unique experts/step {mean_uniq:.1f})")

    # Per-kernel durations on the launch stream (eager pass, events between the launches).
    kt = kernel_times(torch, ops, lib, ws, x, layers, logits, sel, wts, out, args, stream, n_draws)
    gu_bytes_launch = (mean_uniq + 1) * 2 * proj_bytes(H, I, args.bits)
    gu_us = kt["moe_gate_up"]
    roofline = {"bound": "hbm", "kernel": "moe_gate_up",
                "achieved": round(gu_bytes_launch / (gu_us * 1e-6) / 1e9, 1),
                "peak": PEAK_HBM, "unit": "GB/s",
                "frac": round(gu_bytes_launch / (gu_us * 1e-6) / 1e9 / PEAK_HBM, 4),
                "traffic": measured_traffic(T, args.bits),
                "algorithmic_bytes_per_launch": int(gu_bytes_launch),
                "avg_launch_us": round(gu_us, 3)}

    result = {
        "metric": METRIC, "value": round(gbps, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps,
        "warmup": args.warmup, "ms_per_step": round(us_step / 1e3, 6), "us_per_layer": round(us_step, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic (seeded uniform trellis, +-1 suh, +-U(0.5,1.5)/sqrt(H) svh, N(0,1) logits, bf16 N(0,1) x)",
        "config": {"workload": f"DSv3 MoE layer decode, {T} token(s), {args.bits:g} bpw EXL3 "
                               f"(BASELINE configs[{1 if T == 1 else 2}])", "routing": args.routing,
                   "unique_experts_per_step": round(mean_uniq, 2),
                   "hidden": H, "inter": I, "experts": E, "shared": 1, "topk": TOPK, "tokens": T,
                   "bits": args.bits, "layers_cycled": args.layers, "graph": graph is not None,
                   "ksplit_gu": ws_ks(ws, 0), "ksplit_down": ws_ks(ws, 1)},
        "step_bytes": int(step_bytes), "frac_hbm_step": round(gbps / PEAK_HBM, 4),
        "kernel_us": {k: round(v, 3) for k, v in kt.items()},
        "roofline": roofline,
    }
    if not args.no_cpu_baseline:
        log("timing the CPU baseline")
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)


COPY_BYTES = 1 << 30


def copy_calibration(torch):
    """A plain device copy of known size: its FETCH_SIZE / WRITE_SIZE per dispatch, against
    COPY_BYTES, is the scale factor applied to the same counters of the MoE kernels."""
    dev = torch.device("cuda", 0)
    src = torch.empty(COPY_BYTES // 4, dtype=torch.int32, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES, "dispatches": 10}), flush=True)


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "moe_gate_up_traffic_dsv3.md")


def measured_traffic(tokens, bits):
    """HBM bytes per moe_gate_up launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, scaled by the copy calibration), or None if this workload has
    not been profiled."""
    import re
    try:
        text = open(TRAFFIC_FILE).read()
    except OSError:
        return None
    m = re.search(rf"^traffic_bytes_per_launch\[tokens={tokens},bits={bits:g}\]:\s*(\d+)", text, flags=re.M)
    return int(m.group(1)) if m else None


def ws_ks(ws, which):
    return ws.shape.ksplit_gu if which == 0 else ws.shape.ksplit_down


def kernel_times(torch, ops, lib, ws, x, layers, logits, sel, wts, out, args, stream, n_draws, n=64):
    """Average duration of each of the five stages, from hipEvents recorded between the launches
    on the launch stream (eager steps cycling the resident layers)."""
    names = ["moe_prepare", "moe_gate_up", "moe_act", "moe_down", "moe_combine"]
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(6)] for _ in range(n)]
    for row in evs:
        for e in row:
            e.record(stream)          # creates the underlying hipEvent
    handles = []
    with torch.cuda.stream(stream):
        for i in range(n):
            l = i % args.layers
            hs = (ctypes.c_void_p * 6)(*[e.cuda_event for e in evs[i]])
            handles.append(hs)
            ops.moe_forward(ws, x, layers.tables[l], out, limit=10.0, bits=args.bits, logits=logits[i % n_draws],
                            sel=sel, weights=wts, shared_ptrs=layers.shared[l], shared_bits=args.bits,
                            events=hs)
    torch.cuda.synchronize()
    acc = [0.0] * 5
    for i in range(8, n):
        for k in range(5):
            acc[k] += evs[i][k].elapsed_time(evs[i][k + 1])
    return {names[k]: acc[k] * 1e3 / (n - 8) for k in range(5)}


if __name__ == "__main__":
    main()
