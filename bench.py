"""MoE layer decode benchmark on one MI355X (BASELINE.json metric).

Workload: one DeepSeek-V3-shape MoE layer decode step with 1 token:
H=7168, 256 routed experts + 1 shared, I=2048, top-8 sigmoid routing from N(0,1) logits,
every expert EXL3 at 4 bpw (uniform random trellis, +-1 suh, +-U(0.5,1.5) svh), bf16 N(0,1)
activations. A step = routing + grouping + rotations + gate/up GEMV + SwiGLU + down GEMV +
slot reduction + shared expert (evamx_moe_forward), inputs resident in HBM.

Cache hygiene: the weights of L layer copies (257 experts each, 5.7 GB per layer at 4 bpw) stay
resident and every step uses the next layer and a fresh routing draw, so a step's 199 MB are
not served from the 256 MiB MALL. Steps are replayed from a hipGraph.

Other configurations (extra lines, same JSON keys):
  --tokens 16                 configs[2]: 16 tokens, per-token-bias routing
  --workload prefill          configs[3]: 512 tokens, Zipf(1.1) routing, per-expert rates {2,3,4,5}
  --workload stack            configs[4]: 58 stacked layers at 2.5 bpw (all 257 x 58 experts
                              resident, ~205 GB), 8 tokens, bf16 residual, one hipGraph per step

Output: one JSON line (value = achieved HBM GB/s over the algorithmic bytes of the step).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE layer decode µs + achieved HBM GB/s (DSv3 shape, 4bpw EXL3, 1/16 tok)"
PEAK_HBM = 8000.0         # GB/s, MI355X
PEAK_MFMA_F16 = 2500.0    # TFLOP/s, MI355X dense fp16
H, I, E, TOPK = 7168, 2048, 256, 8
STACK_DOWN_SCALE = 0.25   # down-projection svh multiplier of the stacked workload (see DeviceLayers)


def tile_u16(bits):
    b = float(bits)
    return 16 * int(b) + 8 if b != int(b) else 16 * int(b)


def proj_bytes(n_in, n_out, bits):
    return n_in * n_out * bits / 8 + 2 * (n_in + n_out)


def expert_bytes(bits, hidden=H, inter=I):
    return 2 * proj_bytes(hidden, inter, bits) + proj_bytes(inter, hidden, bits)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class DeviceLayers:
    """L layers x (E routed + 1 shared) experts, all resident, with [9, E] pointer tables.

    ``rates``: one rate for every expert, or a callable (layer, expert) -> rate for mixed
    rates (then ``k2[l]`` is the layer's uint8 [E] table of 2 x bits; the shared expert keeps
    ``shared_bits``). ``down_scale`` multiplies the down projections' svh (a stack of layers
    without norms keeps its residual stream O(1) only if each layer's output is small: SwiGLU
    makes the output quadratic in the input, and fp16 gate/up outputs overflow otherwise)."""

    def __init__(self, torch, dev, n_layers, rates, hidden=H, inter=I, n_experts=E, seed=1234, shared_bits=None,
                 down_scale=1.0):
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        self.n = n_experts + 1
        if callable(rates):
            rate_of = rates
            self.mixed = True
        else:
            rate_of = (lambda l, e, r=float(rates): r)
            self.mixed = False
        sb = float(shared_bits) if shared_bits is not None else None
        self.rates = [[float(rate_of(l, e)) if e < n_experts or sb is None else sb for e in range(self.n)]
                      for l in range(n_layers)]
        tiles_gu = (hidden // 16) * (inter // 16)        # tiles per projection (all three equal)
        self.tiles_gu, self.hidden, self.inter = tiles_gu, hidden, inter
        offs, total = [], 0
        for l in range(n_layers):
            row = []
            for e in range(self.n):
                row.append(total)
                total += 3 * tiles_gu * tile_u16(self.rates[l][e])
            offs.append(row)
        self.offs = offs
        log(f"allocating {total * 2 / 1e9:.1f} GB of trellis for {n_layers} layer(s)")
        self.trellis = torch.empty(total, dtype=torch.int16, device=dev)
        chunk = 1 << 28
        for s in range(0, total, chunk):
            self.trellis[s:s + chunk].random_(-32768, 32768, generator=g)
        vec = max(hidden, inter)
        self.suh = (torch.randint(0, 2, (n_layers, self.n, 3, vec), generator=g, device=dev) * 2 - 1).half()
        mag = torch.rand((n_layers, self.n, 3, vec), generator=g, device=dev) + 0.5
        sign = torch.randint(0, 2, (n_layers, self.n, 3, vec), generator=g, device=dev) * 2 - 1
        mag[:, :, 2] *= down_scale
        self.svh = (mag * sign / (hidden ** 0.5)).half()
        del mag, sign
        base_t = self.trellis.data_ptr()
        base_su = self.suh.data_ptr()
        base_sv = self.svh.data_ptr()
        self.tables, self.shared, self.k2 = [], [], []
        for l in range(n_layers):
            rows = [[0] * n_experts for _ in range(9)]
            sh = [0] * 9
            for e in range(self.n):
                pe = tiles_gu * tile_u16(self.rates[l][e])
                ptrs = []
                for p in range(3):
                    k = (l * self.n + e) * 3 + p
                    ptrs += [base_t + 2 * (offs[l][e] + p * pe), base_su + 2 * k * vec, base_sv + 2 * k * vec]
                if e < n_experts:
                    for r in range(9):
                        rows[r][e] = ptrs[r]
                else:
                    sh = ptrs
            self.tables.append(torch.tensor(rows, dtype=torch.int64, device=dev))
            self.shared.append(sh)
            self.k2.append(torch.tensor([int(round(2 * r)) for r in self.rates[l][:n_experts]],
                                        dtype=torch.uint8, device=dev) if self.mixed else None)

    def expert_parts(self, torch, l, e):
        """Host copies of expert e of layer l (e = -1: the shared expert):
        ((trellis, suh, svh) for gate, up, down) as CPU tensors, exactly the bytes the GPU reads."""
        e = self.n - 1 if e < 0 else e
        tu = tile_u16(self.rates[l][e])
        pe = self.tiles_gu * tu
        parts = []
        for p, (n_in, n_out) in enumerate(((self.hidden, self.inter), (self.hidden, self.inter),
                                           (self.inter, self.hidden))):
            t0 = self.offs[l][e] + p * pe
            tr = self.trellis[t0:t0 + pe].view(n_in // 16, n_out // 16, tu).cpu()
            parts.append((tr, self.suh[l, e, p, :n_in].cpu(), self.svh[l, e, p, :n_out].cpu()))
        return tuple(parts)

    def step_bytes(self, l, experts):
        """Algorithmic weight bytes of layer l for the given routed experts plus the shared one."""
        return sum(expert_bytes(self.rates[l][e]) for e in experts) + expert_bytes(self.rates[l][-1])

    def gate_up_bytes(self, l, experts):
        return sum(2 * proj_bytes(H, I, self.rates[l][e]) for e in list(experts) + [self.n - 1])

    def down_bytes(self, l, experts):
        return sum(proj_bytes(I, H, self.rates[l][e]) for e in list(experts) + [self.n - 1])


def cpu_info(torch):
    """Host description for the CPU baseline: lscpu's model name, torch version and threading."""
    model = ""
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        model = next((l.split(":", 1)[1].strip() for l in out.splitlines() if l.startswith("Model name")), "")
    except Exception:
        pass
    if not model:
        try:
            model = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name"))
        except Exception:
            pass
    return {"cpu_model": model, "torch": torch.__version__, "torch_threads": torch.get_num_threads(),
            "mkl": bool(torch.backends.mkl.is_available()), "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS")}


def cpu_baseline(torch, layers, ls, x_dev, logits_list, tokens, limit, what, runs=5, warmups=2, scale=1):
    """The PyTorch-CPU restatement (oracle/torch_cpu.py) on the host cores, on the GPU step's own
    inputs: the first ``tokens`` rows of the step's activations (cast to fp16 as Block.experts
    does) and, for each layer of ``ls`` in turn, its logits, routed on the CPU (sigmoid top-8),
    through the experts of that layer copied from HBM (the routed experts those tokens pick and
    the shared expert); with several layers each layer's output is added to the stream that
    feeds the next. ``warmups`` untimed runs (0: one projection decode warms the allocator and
    the thread pool instead), then the median of ``runs`` runs; GB/s over the same algorithmic
    bytes as the GPU line. ``scale``: the number of such samples in the GPU step (the seconds
    per step estimate is scale times the sample's)."""
    from oracle import torch_cpu

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    x0 = x_dev[:tokens].float().cpu().half().float()
    plans = []
    nbytes = 0
    for l, z_dev in zip(ls, logits_list):
        z = z_dev[:tokens].float().cpu()
        idx, _ = torch_cpu.route_sigmoid(z, TOPK)
        used = sorted(set(idx.reshape(-1).tolist()))
        experts = {e: layers.expert_parts(torch, l, e) for e in used}
        shared = layers.expert_parts(torch, l, -1)
        decs = {}
        for e in used + [-1]:
            rate = layers.rates[l][e if e >= 0 else layers.n - 1]
            decs.setdefault(rate, torch_cpu.Decoder(rate))
        dec = {e: decs[layers.rates[l][e if e >= 0 else layers.n - 1]] for e in used + [-1]}
        plans.append((z, experts, shared, dec, len(used)))
        nbytes += layers.step_bytes(l, used) + tokens * (H * 2 + E * 4 + H * 4)

    def run():
        h = x0
        for z, experts, shared, dec, _ in plans:
            i, w = torch_cpu.route_sigmoid(z, TOPK)
            y = torch_cpu.moe_layer(h, i, w, experts, shared, dec, limit)
            h = (h + y).half().float() if len(plans) > 1 else y
        return h

    if warmups:
        for _ in range(warmups):
            run()
    else:
        z, experts, shared, dec, _ = plans[0]
        tr, suh, svh = shared[0]
        dec[-1].dequant(tr)
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t = sorted(times)[len(times) // 2]
    counts = " + ".join(f"{p[4]}" for p in plans)
    layer_txt = f"layer {ls[0]}" if len(ls) == 1 else f"layers {', '.join(str(l) for l in ls)}"
    runs_txt = (f"median of {runs} runs after {warmups} warm-ups" if warmups
                else f"{'median of ' + str(runs) + ' runs' if runs > 1 else 'one run'} after a warm-up decode")
    res = {"value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
           "sample": f"{what}: {tokens} token(s), {counts} routed experts + the shared expert of {layer_txt} "
                     f"({nbytes / 1e6:.1f} MB), routing included; {runs_txt} ({t:.2f} s per run)",
           "seconds_per_sample": round(t, 3), "runs_s": [round(v, 3) for v in times]}
    if scale != 1:
        res["samples_per_step"] = scale
        res["seconds_per_step_estimate"] = round(t * scale, 2)
    res.update(cpu_info(torch))
    return res


# ---------------------------------------------------------------------------------------------
# rocprofv3 CSV -> markdown summaries (the tables under profiles/ are printed by these).

STAGES = (("prepare", ("moe_prepare", "moe_route", "moe_group", "moe_rotate", "moe_gate_kernel")),
          ("gate/up", ("moe_gate_up",)), ("act", ("moe_act",)), ("down", ("moe_down",)),
          ("combine", ("moe_combine",)))


def kernel_short_name(name):
    """'void evamx::moe_gate_up_mfma_kernel<1>(evamx::MoeParams)' -> 'moe_gate_up_mfma_kernel<1>'."""
    import re
    n = name.strip()
    m = re.match(r"_ZN5evamx(\d+)", n)          # left mangled by the profiler: length-prefixed name
    if m:
        i = m.end()
        ident = n[i:i + int(m.group(1))]
        targs = re.match(r"I((?:Li-?\d+E)+)E", n[i + len(ident):])
        if targs:
            ident += "<" + ", ".join(re.findall(r"Li(-?\d+)E", targs.group(1))) + ">"
        return ident
    if n.startswith("void "):
        n = n[5:]
    depth, cut = 0, len(n)
    for i, ch in enumerate(n):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            cut = i
            break
    n = n[:cut]
    return re.sub(r"^(evamx::|at::native::|\(anonymous namespace\)::)+", "", n)


def stage_of(short):
    for stage, prefixes in STAGES:
        if short.startswith(prefixes):
            return stage
    return None


def summarize_trace(path, skip=0):
    """Per-kernel dispatch count and durations (µs) of a rocprofv3 --kernel-trace CSV, evamx
    kernels only, after dropping each kernel's first ``skip`` dispatches (warm-up), and the time
    per forward of each MoE stage (forwards = dispatches of the combine stage). A stage's time is
    the wall-clock span of each of its occurrences (consecutive dispatches of the stage in start
    order, from the first start to the last end), so two kernels of one stage that run
    concurrently count once."""
    import csv
    import collections
    durs = collections.defaultdict(list)
    events = []
    for row in csv.DictReader(open(path)):
        short = kernel_short_name(row["Kernel_Name"])
        if not row["Kernel_Name"].strip().startswith(("void evamx::", "evamx::", "_ZN5evamx")):
            continue
        t0, t1 = int(row["Start_Timestamp"]), int(row["End_Timestamp"])
        durs[short].append((t1 - t0) / 1e3)
        events.append((t0, t1, stage_of(short)))
    lines = ["| kernel | dispatches | avg µs | median µs | min µs | max µs |", "|---|---|---|---|---|---|"]
    n_fwd = 0
    for k in sorted(durs):
        d = durs[k][skip:] or durs[k]
        lines.append(f"| {k} | {len(d)} | {sum(d) / len(d):.2f} | {median(d):.2f} | {min(d):.2f} | {max(d):.2f} |")
        if stage_of(k) == "combine":
            n_fwd += len(d)
    stage_tot = collections.defaultdict(float)
    events.sort()
    i = 0
    while i < len(events):
        t0, t1, st = events[i]
        j = i + 1
        while j < len(events) and events[j][2] == st:
            t1 = max(t1, events[j][1])
            j += 1
        if st:
            stage_tot[st] += (t1 - t0) / 1e3
        i = j
    # forward wall time: from a forward's first MoE kernel start to the end of its combine
    fwd_spans, first = [], None
    for t0, t1, st in events:
        if not st:
            continue
        if first is None:
            first = t0
        if st == "combine":
            fwd_spans.append((t1 - first) / 1e3)
            first = None
    if n_fwd:
        lines += ["", f"per forward ({n_fwd} forwards; stage spans, concurrent kernels counted once): " + ", ".join(
            f"{st} {stage_tot[st] / n_fwd:.2f} µs" for st, _ in STAGES if st in stage_tot)]
    if fwd_spans:
        lines.append(f"forward wall time (first MoE kernel start to combine end): median {median(fwd_spans):.2f} µs "
                     f"over {len(fwd_spans)} forwards (stages that overlap across streams make the stage spans "
                     f"add up to more)")
    return "\n".join(lines)


def _pmc_rows(path):
    import csv
    import collections
    vals = collections.defaultdict(lambda: collections.defaultdict(float))
    for row in csv.DictReader(open(path)):
        key = (kernel_short_name(row["Kernel_Name"]), int(row["Dispatch_Id"]))
        vals[row["Counter_Name"]][key] += float(row["Counter_Value"])
    return vals


def summarize_pmc(paths, calib_paths, copy_bytes=1 << 30, key=None):
    """FETCH_SIZE / WRITE_SIZE (KiB per dispatch) of rocprofv3 --pmc CSVs, each counter scaled by
    the factor that makes the copy kernel of ``calib_paths`` (``bench.py --copy-calibration``:
    ``copy_bytes`` read and written per dispatch) read and write exactly that; per evamx kernel
    and per MoE stage and forward. With ``key`` also prints the gate/up stage's bytes per forward
    as ``traffic_bytes_per_launch[key]: N`` (the line bench.py reads)."""
    import collections
    factor = {}
    lines = ["| counter | copy kernel KiB per dispatch | expected KiB | scale factor |", "|---|---|---|---|"]
    for cp in calib_paths:
        for counter, per in _pmc_rows(cp).items():
            v = [x for (k, _), x in per.items() if "copyBuffer" in k]
            if v:
                kib = sum(v) / len(v)
                factor[counter] = copy_bytes / 1024 / kib
                lines.append(f"| {counter} | {kib:.0f} | {copy_bytes // 1024} | {factor[counter]:.4f} |")
    per_kernel = collections.defaultdict(dict)
    for p in paths:
        for counter, per in _pmc_rows(p).items():
            by_k = collections.defaultdict(list)
            for (k, _), x in per.items():
                if stage_of(k):
                    by_k[k].append(x)
            for k, xs in by_k.items():
                per_kernel[k][counter] = xs
    counters = sorted({c for d in per_kernel.values() for c in d})
    lines += ["", "| kernel | dispatches | " + " | ".join(f"{c} KiB" for c in counters) + " | "
              + " | ".join(f"scaled {c} MB" for c in counters) + " |",
              "|---|---|" + "---|" * (2 * len(counters))]
    stage_bytes = collections.defaultdict(float)
    n_fwd = 0
    for k in sorted(per_kernel):
        d = per_kernel[k]
        n = max(len(v) for v in d.values())
        avg = {c: sum(d[c]) / len(d[c]) for c in d}
        lines.append(f"| {k} | {n} | " + " | ".join(f"{avg.get(c, 0):.0f}" for c in counters) + " | "
                     + " | ".join(f"{avg.get(c, 0) * 1024 * factor.get(c, 1.0) / 1e6:.2f}" for c in counters) + " |")
        st = stage_of(k)
        stage_bytes[st] += sum(sum(d[c]) * 1024 * factor.get(c, 1.0) for c in d)
        if st == "combine":
            n_fwd = max(n_fwd, n)
    if n_fwd:
        lines += ["", f"HBM bytes per forward by stage (scaled counters summed, {n_fwd} forwards): " + ", ".join(
            f"{st} {stage_bytes[st] / n_fwd:.0f}" for st, _ in STAGES if st in stage_bytes)]
        if key:
            lines.append(f"traffic_bytes_per_launch[{key}]: {stage_bytes['gate/up'] / n_fwd:.0f}")
    return "\n".join(lines)


def summarize_counters(paths):
    """Average per dispatch of every counter in rocprofv3 --pmc CSVs (any counters, e.g. the SQ
    instruction and wait counters), per evamx kernel (measurement kernels included), with the
    ratios the counters present allow: VALU instructions per wave, and the share of wave cycles
    spent issuing VALU (SQ_ACTIVE_INST_VALU) and waiting (SQ_WAIT_INST_ANY)."""
    import collections
    per_kernel = collections.defaultdict(lambda: collections.defaultdict(list))
    for p in paths:
        for counter, per in _pmc_rows(p).items():
            for (k, _), x in per.items():
                if stage_of(k) or k.startswith("bench_"):
                    per_kernel[k][counter].append(x)
    counters = sorted({c for d in per_kernel.values() for c in d})
    ratios = [("VALU insts / wave", "SQ_INSTS_VALU", "SQ_WAVES"),
              ("active VALU / wave cycles", "SQ_ACTIVE_INST_VALU", "SQ_WAVE_CYCLES"),
              ("wait / wave cycles", "SQ_WAIT_INST_ANY", "SQ_WAVE_CYCLES")]
    ratios = [r for r in ratios if r[1] in counters and r[2] in counters]
    lines = ["| kernel | dispatches | " + " | ".join(counters) + "".join(f" | {r[0]}" for r in ratios) + " |",
             "|---|---|" + "---|" * (len(counters) + len(ratios))]
    for k in sorted(per_kernel):
        d = per_kernel[k]
        avg = {c: sum(v) / len(v) for c, v in d.items()}
        n = max(len(v) for v in d.values())
        row = f"| {k} | {n} | " + " | ".join(f"{avg.get(c, 0):.4g}" for c in counters)
        for _, num, den in ratios:
            row += f" | {avg[num] / avg[den]:.4g}" if avg.get(den) else " | -"
        lines.append(row + " |")
    return "\n".join(lines)


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", choices=("layer", "stack", "prefill", "linear"), default="layer",
                    help="layer: one decode layer (configs[1] at 1 token, configs[2] at 16); stack: configs[4], "
                         "58 stacked layers at 2.5 bpw, 8 tokens, one hipGraph; prefill: configs[3], 512 tokens, "
                         "Zipf routing, per-expert rates {2,3,4,5}; linear: configs[0], one EXL3 linear "
                         "2048 -> 7168 at 4 bpw, 1 token, over 64 resident copies in one graph")
    ap.add_argument("--tokens", type=int, default=None)
    ap.add_argument("--bits", type=float, default=None)
    ap.add_argument("--layers", type=int, default=None)
    ap.add_argument("--graph-steps", type=int, default=8)
    ap.add_argument("--ksplit-gu", type=int, default=0)
    ap.add_argument("--ksplit-down", type=int, default=0)
    ap.add_argument("--routing", choices=("plain", "skewed"), default=None,
                    help="N(0,1) logits, or config 3's per-token bias (default: plain at 1 token, skewed above)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--mode", choices=("strict", "fast"), default="strict",
                    help="strict (default, as the reference's DS41_STRICT_BATCH): calls of up to 64 tokens give "
                         "every token a one-token call's bits; fast: the geometry is chosen per call size")
    ap.add_argument("--also-tokens", type=int, default=16,
                    help="with the default 1-token layer, also measure this many tokens (configs[2]) and report "
                         "it under \"also\" in the same line (0: off)")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--clock-warmup-ms", type=float, default=300.0,
                    help="untimed replays for at least this long before the warm-up steps (0: none)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 1 GiB device copy (the reference kernel for FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--summarize-trace", metavar="CSV",
                    help="print the markdown summary of a rocprofv3 kernel_trace.csv and exit (no GPU)")
    ap.add_argument("--summarize-pmc", metavar="CSV", nargs="+",
                    help="print the markdown summary of rocprofv3 --pmc counter_collection.csv files and exit")
    ap.add_argument("--calibration", metavar="CSV", nargs="*", default=[],
                    help="with --summarize-pmc: the counter CSVs of a --copy-calibration run")
    ap.add_argument("--traffic-key", default=None, help="with --summarize-pmc: e.g. tokens=1,bits=4,mode=strict")
    ap.add_argument("--summarize-counters", metavar="CSV", nargs="+",
                    help="print per-kernel averages of any rocprofv3 --pmc counters and exit (no GPU)")
    ap.add_argument("--skip-dispatches", type=int, default=0, help="with --summarize-trace: warm-up dispatches")
    args = ap.parse_args()
    defaults = {"layer": (1, 4.0, 4), "stack": (8, 2.5, 58), "prefill": (512, None, 2), "linear": (1, 4.0, 64)}[args.workload]
    if args.tokens is None:
        args.tokens = defaults[0]
    if args.bits is None:
        args.bits = defaults[1]
    if args.layers is None:
        args.layers = defaults[2]
    return args


def main():
    args = parse_args()
    if args.summarize_trace:
        print(summarize_trace(args.summarize_trace, args.skip_dispatches))
        return
    if args.summarize_counters:
        print(summarize_counters(args.summarize_counters))
        return
    if args.summarize_pmc:
        print(summarize_pmc(args.summarize_pmc, args.calibration, key=args.traffic_key))
        return
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (the expert path "
              "shards by experts across GPUs, which one GPU cannot show); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_calibration:
        copy_calibration(torch)
        return
    if args.workload == "stack":
        result = run_stack(torch, args)
    elif args.workload == "linear":
        result = run_linear(torch, args)
    else:
        result = run_layer(torch, args)
        if args.workload == "layer" and args.tokens == 1 and args.also_tokens > 0:
            # the metric covers 1 and 16 tokens: the 16-token point rides along in the same line
            # (same mode, with its own CPU baseline), and both points in the other mode beside them
            import copy

            other = "fast" if args.mode == "strict" else "strict"
            keys = ("us_per_layer", "value", "unit", "step_bytes", "frac_hbm_step", "kernel_us", "roofline")
            runs = {}
            for mode, T in ((args.mode, args.also_tokens), (other, 1), (other, args.also_tokens)):
                sub = copy.copy(args)
                sub.tokens, sub.routing, sub.mode = T, None, mode
                sub.no_cpu_baseline = args.no_cpu_baseline or mode != args.mode
                runs[mode, T] = run_layer(torch, sub)
            r2 = runs[args.mode, args.also_tokens]
            result["also"] = {k: r2[k] for k in keys + (("cpu_baseline",) if "cpu_baseline" in r2 else ())}
            result["also"]["config"] = r2["config"]["workload"]
            result["also"]["mode"] = r2["config"]["mode"]
            result["modes"] = {
                "headline": args.mode,
                "note": "strict: calls of up to strict_rows tokens give every token the bits of a one-token "
                        "call (the reference's default DS41_STRICT_BATCH); at 1 token both modes run the same "
                        "kernels with the same splits",
                args.mode: {"us_per_layer_1": result["us_per_layer"], f"us_per_layer_{args.also_tokens}": r2["us_per_layer"]},
                other: {"us_per_layer_1": runs[other, 1]["us_per_layer"],
                        f"us_per_layer_{args.also_tokens}": runs[other, args.also_tokens]["us_per_layer"],
                        f"kernel_us_{args.also_tokens}": runs[other, args.also_tokens]["kernel_us"]},
            }
    print(json.dumps(result), flush=True)


def make_logits(torch, g, dev, n_draws, T, routing):
    logits = torch.randn((n_draws, T, E), generator=g, device=dev)
    if routing == "skewed":
        # config 3: per-token random bias so expert loads span 0..T (2 hot experts +6 for every
        # token, 6 warm experts +3 for a per-token coin flip, a fresh draw of both per step)
        for i in range(n_draws):
            perm = torch.randperm(E, generator=g, device=dev)
            logits[i][:, perm[:2]] += 6.0
            coin = torch.randint(0, 2, (T, 6), generator=g, device=dev).float()
            logits[i][:, perm[2:8]] += 3.0 * coin
    elif routing == "zipf":
        # config 4: Zipf(1.1) over a random expert permutation, 8 distinct picks per token
        # (log p + Gumbel noise: its top-k is a draw without replacement with probabilities p)
        ranks = torch.arange(1, E + 1, dtype=torch.float64, device=dev)
        logp = torch.log(ranks ** -1.1 / (ranks ** -1.1).sum())
        for i in range(n_draws):
            perm = torch.randperm(E, generator=g, device=dev)
            lp = torch.empty(E, dtype=torch.float64, device=dev)
            lp[perm] = logp
            u = torch.rand((T, E), generator=g, device=dev, dtype=torch.float64).clamp_(1e-300, 1.0)
            logits[i] = (lp[None, :] - torch.log(-torch.log(u))).float()
    return logits


MIN_REPLAYS = 20


def clock_warmup(torch, stream, replay, min_ms, unit=1):
    """Untimed replays of the measured graph(s), ``unit`` at a time with a synchronisation after
    each batch, until ``min_ms`` of wall time has passed. The GPU's clocks rise over the first
    hundreds of milliseconds of sustained load: after a few warm-up steps alone the timed steps
    run below the steady-state rate (one-token layer, one box, three runs each: 69.1-72.3 us per
    step after 5 warm-up steps, 63.7-65.1 us after ~280 ms of replays). Returns (replays, ms)."""
    if min_ms <= 0:
        return 0, 0.0
    t0 = time.perf_counter()
    n = 0
    batch = unit * max(1, 8 // unit)
    with torch.cuda.stream(stream):
        while True:
            for _ in range(batch):
                replay()
            n += batch
            torch.cuda.synchronize()
            ms = (time.perf_counter() - t0) * 1e3
            if ms >= min_ms:
                return n, ms


def timed_replays(torch, stream, replay, n, warm):
    """``warm`` untimed calls of ``replay`` (one graph replay), then ``n`` timed ones on
    ``stream``, each between its own pair of consecutive events. Returns (ms of each replay, ms
    of all n from the first event to the last)."""
    with torch.cuda.stream(stream):
        for _ in range(warm):
            replay()
    torch.cuda.synchronize()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    with torch.cuda.stream(stream):
        evs[0].record(stream)
        for i in range(n):
            replay()
            evs[i + 1].record(stream)
    torch.cuda.synchronize()
    return [evs[i].elapsed_time(evs[i + 1]) for i in range(n)], evs[0].elapsed_time(evs[n])


def strict_rows_for(mode, T):
    """strict_rows of the benchmark's workspace: the call's own rows in strict mode (within the
    strict bound of 64 rows and 256 slots), else 0."""
    return T if mode == "strict" and T <= 64 and T * TOPK <= 256 else 0


_LAYERS = {}


def resident_layers(torch, dev, n_layers, bits, **kw):
    """DeviceLayers of a uniform rate, kept across the runs of one bench process (the extra
    lines reuse the headline line's resident weights instead of allocating them again)."""
    key = (n_layers, bits, tuple(sorted(kw.items())))
    if key not in _LAYERS:
        _LAYERS.clear()
        _LAYERS[key] = DeviceLayers(torch, dev, n_layers, bits, **kw)
    return _LAYERS[key]


def median(v):
    v = sorted(v)
    n = len(v)
    return v[n // 2] if n % 2 else 0.5 * (v[n // 2 - 1] + v[n // 2])


def replay_stats(ms, steps_per_replay):
    """Per-step figures from per-replay times: the median (the reported value), the mean over
    the whole timed region, and the spread."""
    per = [m / steps_per_replay for m in ms]
    return {"replays": len(ms), "steps_per_replay": steps_per_replay, "median_ms": median(per),
            "mean_ms": sum(per) / len(per), "min_ms": min(per), "max_ms": max(per)}


def run_layer(torch, args):
    """One MoE layer per step, cycling resident layers."""
    from eva_amd import ops
    from eva_amd._lib import lib

    dev = torch.device("cuda", 0)
    T = args.tokens
    prefill = args.workload == "prefill"
    if args.routing is None:
        args.routing = "zipf" if prefill else ("plain" if T == 1 else "skewed")
    if prefill:
        rng_rates = torch.Generator().manual_seed(4321)
        rate_tab = [[float((2, 3, 4, 5)[int(v)]) for v in torch.randint(0, 4, (E,), generator=rng_rates)]
                    for _ in range(args.layers)]
        layers = DeviceLayers(torch, dev, args.layers, lambda l, e: rate_tab[l][e], shared_bits=4.0)
    else:
        layers = resident_layers(torch, dev, args.layers, args.bits)
    g = torch.Generator(device=dev)
    g.manual_seed(99)
    # The step sequence cycles C = --graph-steps (layer, routing draw) pairs (one for prefill).
    # Exactly --steps steps are timed: graph replays of G steps, G the largest divisor of both,
    # the C/G graphs of the cycle replayed in turn, so the timed draws do not depend on --steps.
    C = 1 if prefill else args.graph_steps
    G = math.gcd(max(1, args.steps), C)
    reps = max(1, args.steps) // G
    n_graphs = C // G
    n_draws = max(C, args.layers) * 2
    logits = make_logits(torch, g, dev, n_draws, T, args.routing)
    x = torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16)
    strict_rows = strict_rows_for(args.mode, T)
    ws = ops.MoeWorkspace(dev, rows_max=T, hidden=H, inter=I, topk=TOPK, n_local=E, has_shared=True,
                          ksplit_gu=args.ksplit_gu, ksplit_down=args.ksplit_down, strict_rows=strict_rows)
    sel = torch.empty(T, TOPK, dtype=torch.int64, device=dev)
    wts = torch.empty(T, TOPK, dtype=torch.float32, device=dev)
    out = torch.empty(T, H, dtype=torch.float32, device=dev)
    shared_bits = 4.0 if prefill else args.bits

    def step(i, events=None):
        l = i % args.layers
        ops.moe_forward(ws, x, layers.tables[l], out, limit=10.0, bits=None if prefill else args.bits,
                        k2_per_expert=layers.k2[l], logits=logits[i % n_draws], sel=sel, weights=wts,
                        shared_ptrs=layers.shared[l], shared_bits=shared_bits, events=events)

    # experts touched per step (for the algorithmic bytes), from the same routing draws
    touched = []
    for i in range(n_draws):
        step(i)
        touched.append(sorted(set(sel.reshape(-1).tolist())))
    torch.cuda.synchronize()
    if not torch.isfinite(out).all():
        raise RuntimeError("non-finite layer output")
    if int(ws.flags().cpu()[0]) != 0:
        raise RuntimeError(f"device error flags {int(ws.flags().cpu()[0])}")
    act_bytes = T * H * 2 + T * E * 4 + T * H * 4

    stream = torch.cuda.Stream(device=dev)
    graphs = []
    if not args.no_graph:
        with torch.cuda.stream(stream):
            for i in range(C):
                step(i)
            torch.cuda.synchronize()
            for j in range(n_graphs):
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=stream):
                    for i in range(j * G, (j + 1) * G):
                        step(i)
                graphs.append(graph)
    steps = reps * G
    timed = [(r % n_graphs) * G + i for r in range(reps) for i in range(G)]      # cycle positions timed
    step_bytes = sum(layers.step_bytes(i % args.layers, touched[i % n_draws]) for i in timed) / steps + act_bytes
    mean_uniq = sum(len(touched[i % n_draws]) for i in timed) / steps
    counter = [0]

    def replay():
        j = counter[0] % n_graphs
        counter[0] += 1
        if graphs:
            graphs[j].replay()
        else:
            for i in range(j * G, (j + 1) * G):
                step(i)

    warm = max(1, -(-args.warmup // G))
    warm += (-warm) % n_graphs                      # the timed replays start at the cycle's first graph
    cw = clock_warmup(torch, stream, replay, args.clock_warmup_ms, n_graphs)
    ms, total_ms = timed_replays(torch, stream, replay, reps, warm)
    st = replay_stats(ms, G)
    us_step = st["median_ms"] * 1e3
    gbps = step_bytes / (us_step * 1e-6) / 1e9
    log(f"{steps} steps in {reps} replays: median {us_step:.2f} us/step (mean {st['mean_ms'] * 1e3:.2f}), "
        f"{gbps:.1f} GB/s (unique experts/step {mean_uniq:.1f})")

    # Per-kernel durations on the launch stream (eager pass, events between the launches).
    n_ev = 16 if prefill else 64
    # one-token calls route inside the gate/up launch: their prepare stage has no kernel
    kt = kernel_times(torch, stream, step, n_ev, skip=2 if prefill else 8,
                      kernelless=("moe_prepare",) if T == 1 else ())
    gu_bytes_launch = sum(layers.gate_up_bytes(i % args.layers, touched[i % n_draws]) for i in range(n_ev)) / n_ev
    roofline = gate_up_roofline(gu_bytes_launch, kt["moe_gate_up"],
                                measured_traffic(T, args.bits, "strict" if strict_rows else "fast"))
    if prefill:
        roofline["decode_alu_ceiling"] = decode_ceiling(ops, (2.0, 3.0, 4.0, 5.0))
        # MFMA utilisation of the gate/up GEMM: 2 * H * I flops per row and projection
        flops = 2 * H * I * 2 * (T * TOPK + T)
        roofline["mfma"] = {"kernel": "moe_gate_up", "achieved": round(flops / (kt["moe_gate_up"] * 1e-6) / 1e12, 1),
                            "peak": PEAK_MFMA_F16, "unit": "TFLOP/s",
                            "frac": round(flops / (kt["moe_gate_up"] * 1e-6) / 1e12 / PEAK_MFMA_F16, 4),
                            "flops_per_launch": flops}
    else:
        roofline["decode_alu_ceiling"] = decode_ceiling(ops, (args.bits,), roofline["achieved"])
        if T == 1 and args.bits == 4.0:
            roofline["read_floor"] = read_floor(torch, ops, H, I, TOPK + 1, 2, roofline["achieved"])
            # the down launch beside it: its own bytes, decode ceiling and read floor
            d_bytes = sum(layers.down_bytes(i % args.layers, touched[i % n_draws]) for i in range(n_ev)) / n_ev
            d_ach = d_bytes / (kt["moe_down"] * 1e-6) / 1e9
            ceil = roofline["decode_alu_ceiling"]["value"]
            roofline["down"] = {"kernel": "moe_down", "achieved": round(d_ach, 1), "peak": PEAK_HBM, "unit": "GB/s",
                                "frac": round(d_ach / PEAK_HBM, 4), "algorithmic_bytes_per_launch": int(d_bytes),
                                "avg_launch_us": round(kt["moe_down"], 3), "decode_alu_ceiling_frac": round(d_ach / ceil, 4),
                                "read_floor": read_floor(torch, ops, I, H, TOPK + 1, 1, d_ach)}
    cfg_idx = 3 if prefill else (1 if T == 1 else 2)
    rates = "per-expert rates {2,3,4,5} (shared 4)" if prefill else f"{args.bits:g} bpw"
    result = {
        "metric": METRIC, "value": round(gbps, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps,
        "warmup": args.warmup, "clock_warmup": {"replays": cw[0], "ms": round(cw[1], 1)},
        "ms_per_step": round(us_step / 1e3, 6), "us_per_layer": round(us_step, 3),
        "timing": {k: (round(v, 6) if isinstance(v, float) else v) for k, v in st.items()},
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic (seeded uniform trellis, +-1 suh, +-U(0.5,1.5)/sqrt(H) svh, N(0,1) logits, bf16 N(0,1) x)",
        "config": {"workload": f"DSv3 MoE layer {'prefill' if prefill else 'decode'}, {T} token(s), {rates} EXL3 "
                               f"(BASELINE configs[{cfg_idx}])", "routing": args.routing,
                   "unique_experts_per_step": round(mean_uniq, 2),
                   "hidden": H, "inter": I, "experts": E, "shared": 1, "topk": TOPK, "tokens": T,
                   "bits": None if prefill else args.bits, "layers_cycled": args.layers, "graph": bool(graphs),
                   "graph_steps": G, "step_cycle": C,
                   "ksplit_gu": ws.shape.ksplit_gu, "ksplit_down": ws.shape.ksplit_down,
                   "mode": "strict" if strict_rows else "fast", "strict_rows": strict_rows},
        "step_bytes": int(step_bytes), "frac_hbm_step": round(gbps / PEAK_HBM, 4),
        "kernel_us": {k: round(v, 3) for k, v in kt.items()},
        "roofline": roofline,
    }
    if T == 1:
        result["kernel_us_note"] = "1 token: routing runs inside moe_gate_up (no prepare launch)"
    if not args.no_cpu_baseline:
        log("timing the CPU baseline")
        if T == 1:
            result["cpu_baseline"] = cpu_baseline(torch, layers, [0], x, [logits[0]], 1, 10.0,
                                                  "step 0 of the timed sequence (layer 0, routing draw 0)")
        elif not prefill:
            # the whole step (every token, every expert they touch): one run after a warm-up decode
            result["cpu_baseline"] = cpu_baseline(torch, layers, [0], x, [logits[0]], T, 10.0,
                                                  "step 0 of the timed sequence (layer 0, routing draw 0)",
                                                  runs=1, warmups=0)
        else:
            # a bounded sample of the prefill step: its first 32 tokens (about 25 s of CPU work)
            result["cpu_baseline"] = cpu_baseline(torch, layers, [0], x, [logits[0]], 32, 10.0,
                                                  "the first 32 tokens of step 0 (layer 0, routing draw 0) of 512",
                                                  runs=1, warmups=0)
    return result


def run_stack(torch, args):
    """an expert-only decode step through L stacked layers (all 257 x L experts
    resident), 8 tokens, independent routing per layer, bf16 residual add between layers, the
    whole step captured as one hipGraph (a copy of the step's input residual, then L layers)."""
    from eva_amd import ops

    dev = torch.device("cuda", 0)
    T, L, K = args.tokens, args.layers, args.bits
    layers = DeviceLayers(torch, dev, L, K, down_scale=STACK_DOWN_SCALE)
    g = torch.Generator(device=dev)
    g.manual_seed(77)
    logits = torch.randn((L, T, E), generator=g, device=dev)
    h0 = torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16)
    h = h0.clone()
    strict_rows = strict_rows_for(args.mode, T)
    ws = ops.MoeWorkspace(dev, rows_max=T, hidden=H, inter=I, topk=TOPK, n_local=E, has_shared=True,
                          ksplit_gu=args.ksplit_gu, ksplit_down=args.ksplit_down, strict_rows=strict_rows)
    sels = torch.empty(L, T, TOPK, dtype=torch.int64, device=dev)
    wts = torch.empty(L, T, TOPK, dtype=torch.float32, device=dev)

    def layer(l, events=None):
        ops.moe_forward(ws, h, layers.tables[l], None, limit=10.0, bits=K, logits=logits[l], sel=sels[l],
                        weights=wts[l], shared_ptrs=layers.shared[l], shared_bits=K, residual=h, events=events)

    def step():
        h.copy_(h0)
        for l in range(L):
            layer(l)

    step()
    torch.cuda.synchronize()
    if not torch.isfinite(h.float()).all():
        raise RuntimeError("non-finite residual stream")
    h_max = h.float().abs().max().item()
    touched = [sorted(set(sels[l].reshape(-1).tolist())) for l in range(L)]
    step_bytes = sum(layers.step_bytes(l, touched[l]) for l in range(L)) + L * (2 * T * H * 2 + T * E * 4)
    mean_uniq = sum(len(t) for t in touched) / L

    stream = torch.cuda.Stream(device=dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        step()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            step()
    steps = max(1, args.steps)                 # one replay = one step through the L layers

    cw = clock_warmup(torch, stream, graph.replay, args.clock_warmup_ms)
    ms, total_ms = timed_replays(torch, stream, graph.replay, steps, max(1, min(args.warmup, 5)))
    st = replay_stats(ms, 1)
    ms_step = st["median_ms"]
    gbps = step_bytes / (ms_step * 1e-3) / 1e9
    log(f"{steps} graph replays of {L} layers: median {ms_step:.3f} ms/step (mean {st['mean_ms']:.3f}), "
        f"{gbps:.1f} GB/s (unique experts/layer {mean_uniq:.1f})")
    ref = h.clone()
    with torch.cuda.stream(stream):
        graph.replay()
    torch.cuda.synchronize()
    if not torch.equal(ref, h):
        raise RuntimeError("graph replays of the stacked step are not deterministic")

    kt = kernel_times(torch, stream, lambda i, events=None: layer(i % L, events), L, skip=0)
    gu_bytes_launch = sum(layers.gate_up_bytes(l, touched[l]) for l in range(L)) / L
    roofline = gate_up_roofline(gu_bytes_launch, kt["moe_gate_up"], measured_traffic(T, K, "strict" if strict_rows else "fast"))
    roofline["decode_alu_ceiling"] = decode_ceiling(ops, (K,), roofline["achieved"])
    result = {
        "metric": METRIC, "value": round(gbps, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps,
        "warmup": args.warmup, "clock_warmup": {"replays": cw[0], "ms": round(cw[1], 1)},
        "ms_per_step": round(ms_step, 4), "us_per_layer": round(ms_step * 1e3 / L, 3),
        "timing": {k: (round(v, 6) if isinstance(v, float) else v) for k, v in st.items()},
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic (seeded uniform trellis, +-1 suh, +-U(0.5,1.5)/sqrt(H) svh, N(0,1) logits, bf16 N(0,1) h)",
        "config": {"workload": f"DSv3 expert-only decode step, {L} stacked layers, {T} tokens, {K:g} bpw EXL3, "
                               f"bf16 residual, one hipGraph (BASELINE configs[4])",
                   "layers": L, "tokens": T, "bits": K, "resident_weight_gb": round(layers.trellis.numel() * 2 / 1e9, 2),
                   "unique_experts_per_layer": round(mean_uniq, 2), "down_svh_scale": STACK_DOWN_SCALE,
                   "residual_max_abs": round(h_max, 3), "hidden": H, "inter": I, "experts": E,
                   "shared": 1, "topk": TOPK, "mode": "strict" if strict_rows else "fast", "strict_rows": strict_rows},
        "step_bytes": int(step_bytes), "frac_hbm_step": round(gbps / PEAK_HBM, 4),
        "kernel_us": {k: round(v, 3) for k, v in kt.items()},
        "roofline": roofline,
    }
    if T == 1:
        result["kernel_us_note"] = "1 token: routing runs inside moe_gate_up (no prepare launch)"
    if not args.no_cpu_baseline:
        log("timing the CPU baseline")
        # the configuration's own work: 2 layers of the step, scaled by L / 2
        result["cpu_baseline"] = cpu_baseline(torch, layers, [0, 1], h0, [logits[0], logits[1]], T, 10.0,
                                              f"layers 0 and 1 of the stacked step, all {T} tokens (x{L // 2} "
                                              f"for the {L}-layer step)", runs=1, warmups=0, scale=L / 2)
    return result


def run_linear(torch, args):
    """one EXL3 linear 2048 -> 7168 at 4 bpw on 1 token. A call moves 7.4 MB, so it is
    launch-bound: `--layers` resident copies (default 64) are cycled in one graph, and the time per
    call is the graph's time over the calls."""
    from eva_amd import ops

    dev = torch.device("cuda", 0)
    n_in, n_out, T, copies = 2048, 7168, args.tokens, args.layers
    bits = args.bits
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    tu = tile_u16(bits)
    trellis = torch.randint(-32768, 32768, (copies, n_in // 16, n_out // 16, tu), generator=g, device=dev,
                            dtype=torch.int32).to(torch.int16)
    suh = (torch.randint(0, 2, (copies, n_in), generator=g, device=dev) * 2 - 1).to(torch.float16)
    mag = torch.rand((copies, n_out), generator=g, device=dev) + 0.5
    svh = ((torch.randint(0, 2, (copies, n_out), generator=g, device=dev) * 2 - 1) * mag).to(torch.float16)
    x = torch.randn((T, n_in), generator=g, device=dev).to(torch.bfloat16).to(torch.float16)
    out = torch.empty(copies, T, n_out, dtype=torch.float16, device=dev)
    ws = torch.empty(ops.lib().evamx_exl3_linear_workspace_bytes(T, n_in, n_out), dtype=torch.uint8, device=dev)

    def call(i):
        ops.exl3_linear(x, trellis[i], suh[i], svh[i], bits, out=out[i], workspace=ws)

    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        for i in range(copies):
            call(i)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(copies):
                call(i)
    eager = out.clone()
    reps = max(MIN_REPLAYS, -(-args.steps // copies))
    cw = clock_warmup(torch, stream, graph.replay, args.clock_warmup_ms)
    ms, total_ms = timed_replays(torch, stream, graph.replay, reps, max(1, -(-args.warmup // copies)))
    st = replay_stats(ms, copies)
    dt = st["median_ms"] * 1e-3
    if not torch.equal(out, eager):
        raise RuntimeError("graph replays differ from the eager calls")
    nbytes = n_in * n_out * bits / 8 + 2 * (n_in + n_out) + T * 2 * (n_in + n_out)
    gbps = nbytes / dt / 1e9
    result = {
        "metric": METRIC, "value": round(gbps, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": reps * copies, "warmup": args.warmup, "clock_warmup": {"replays": cw[0], "ms": round(cw[1], 1)},
        "ms_per_step": round(dt * 1e3, 6),
        "us_per_call": round(dt * 1e6, 3),
        "timing": {k: (round(v, 6) if isinstance(v, float) else v) for k, v in st.items()}, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16", "data": "synthetic (seeded uniform trellis, +-1 suh, +-U(0.5,1.5) svh, bf16 N(0,1) x)",
        "config": {"workload": f"single EXL3 linear {n_in} -> {n_out}, {bits:g} bpw, {T} token(s), "
                               f"{copies} resident copies in one graph (BASELINE configs[0])",
                   "in": n_in, "out": n_out, "tokens": T, "bits": bits, "copies": copies},
        "step_bytes": int(nbytes), "frac_hbm_step": round(gbps / PEAK_HBM, 4),
        "roofline": {"bound": "hbm", "kernel": "exl3_linear (" + (
                         "1 launch: GEMV with its input rotation, the epilogue in each column group's last workgroup"
                         if T <= 2 else "3 launches: rotation, GEMV, epilogue" if T <= 16
                         else "2 launches: rotation, MFMA tiles with their epilogue") + " per call)",
                     "achieved": round(gbps, 1),
                     "peak": PEAK_HBM, "unit": "GB/s", "frac": round(gbps / PEAK_HBM, 4), "traffic": None},
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_linear_baseline(torch, x, trellis[0], suh[0], svh[0], bits)
    return result


def cpu_linear_baseline(torch, x_dev, trellis_dev, suh_dev, svh_dev, bits):
    """The PyTorch-CPU restatement of the same linear on the GPU run's own inputs (copy 0 of the
    resident weights, the same activations): LUT decode, H128 matmuls, fp32 product. 2 warm-ups,
    then the median of 5 runs."""
    from oracle import torch_cpu

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    tr, suh, svh = trellis_dev.cpu(), suh_dev.cpu(), svh_dev.cpu()
    x = x_dev.float().cpu()
    dec = torch_cpu.Decoder(bits)
    for _ in range(2):
        torch_cpu.linear_forward(x, tr, suh, svh, dec)
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        torch_cpu.linear_forward(x, tr, suh, svh, dec)
        times.append(time.perf_counter() - t0)
    t = sorted(times)[2]
    n_in, n_out = suh.numel(), svh.numel()
    nbytes = n_in * n_out * bits / 8 + 2 * (n_in + n_out) + x.shape[0] * 2 * (n_in + n_out)
    res = {"value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
           "sample": f"copy 0 of the GPU run's {n_in} -> {n_out} linear at {bits:g} bpw on its {x.shape[0]} token(s); "
                     f"median of 5 runs after 2 warm-ups ({t * 1e3:.1f} ms per run)",
           "seconds_per_sample": round(t, 4), "runs_s": [round(v, 4) for v in times]}
    res.update(cpu_info(torch))
    return res


def gate_up_roofline(bytes_launch, us, traffic):
    achieved = bytes_launch / (us * 1e-6) / 1e9
    return {"bound": "hbm", "kernel": "moe_gate_up", "achieved": round(achieved, 1), "peak": PEAK_HBM,
            "unit": "GB/s", "frac": round(achieved / PEAK_HBM, 4), "traffic": traffic,
            "algorithmic_bytes_per_launch": int(bytes_launch), "avg_launch_us": round(us, 3)}


def decode_ceiling(ops, bits_list, achieved_gbps=None, weights=None):
    """Arithmetic bound of the decode GEMV (evamx_bench_decode: the GEMV's per-weight decode and
    dot-product instructions on register-resident words, no memory traffic), as trellis GB/s at
    each rate; with one rate, also the fraction of it the dominant kernel reached."""
    out = {"kernel": "evamx_bench_decode", "unit": "GB/s"}
    per = {}
    for b in bits_list:
        wps = ops.decode_ceiling(b)
        per[f"{b:g}"] = round(wps * b / 8 / 1e9, 1)
    out["value"] = per if len(per) > 1 else next(iter(per.values()))
    if achieved_gbps is not None and len(per) == 1:
        out["frac"] = round(achieved_gbps / out["value"], 4)
    return out


def read_floor(torch, ops, n_in, n_out, units, nproj, achieved_gbps):
    """Memory-side bound of a one-row decode GEMV launch (evamx_bench_read): the launch's own bytes
    in its own shape, without the decode. One-row calls aim their k-split at two waves per SIMD:
    units x nproj (gate/up: 2, down: 1) x n_out/128 column groups x ks waves, ks = that target over
    the per-split items, each wave streaming the 8 * (n_in/128 / ks) k-slices of its split as 1 KiB
    chunks (8 tiles at 4 bits), four in flight. Back-to-back launches over distinct copies of at
    least 1 GiB in total (a repeated buffer of this size would be served partly by the Infinity
    Cache), so the figure includes each launch's ramp and tail but only part of the gap between
    launches."""
    ncg = n_out // 128
    per_split = units * nproj * ncg
    waves_target = torch.cuda.get_device_properties(0).multi_processor_count * 16 // 2
    ks = max(1, waves_target // per_split)
    rows = 8 * ((n_in // 128) // ks)
    waves = per_split * ks
    bps = ops.read_floor(ncg, rows, waves)
    return {"kernel": "evamx_bench_read", "unit": "GB/s", "value": round(bps / 1e9, 1),
            "bytes_per_launch": waves * rows * 1024, "waves": waves, "slices_per_wave": rows,
            "frac": round(achieved_gbps / (bps / 1e9), 4)}


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


def measured_traffic(tokens, bits, mode):
    """HBM bytes per moe_gate_up launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, scaled by the copy calibration), or None if this workload has
    not been profiled in this mode (1-token calls run the same kernels in both modes)."""
    import re
    try:
        text = open(TRAFFIC_FILE).read()
    except OSError:
        return None
    key = "mixed" if bits is None else f"{bits:g}"
    mode = "strict" if tokens == 1 else mode
    m = re.search(rf"^traffic_bytes_per_launch\[tokens={tokens},bits={key},mode={mode}\]:\s*(\d+)", text, flags=re.M)
    return int(m.group(1)) if m else None


def kernel_times(torch, stream, step, n, skip, kernelless=()):
    """Average duration of each of the five stages, from the start timestamp of a stage's first
    kernel to the end timestamp of its last (events taken by the kernel launches themselves on
    the launch stream; eager calls step(i, events)). Stages in ``kernelless`` run inside another
    stage's launch in these calls and record no events (evamx_moe_args.events): reported as 0."""
    names = ["moe_prepare", "moe_gate_up", "moe_act", "moe_down", "moe_combine"]
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(10)] for _ in range(n)]
    for row in evs:
        for e in row:
            e.record(stream)          # creates the underlying hipEvent
    torch.cuda.synchronize()
    handles = []
    with torch.cuda.stream(stream):
        for i in range(n):
            hs = (ctypes.c_void_p * 10)(*[e.cuda_event for e in evs[i]])
            handles.append(hs)
            step(i, events=hs)
    torch.cuda.synchronize()
    acc = [0.0] * 5
    for i in range(skip, n):
        for k in range(5):
            acc[k] += evs[i][2 * k].elapsed_time(evs[i][2 * k + 1])
    return {names[k]: 0.0 if names[k] in kernelless else acc[k] * 1e3 / (n - skip) for k in range(5)}


if __name__ == "__main__":
    main()
