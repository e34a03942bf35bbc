"""Seeded random layer configurations on the GPU against the CPU oracle: shapes off the tested grid
(hidden and intermediate widths of 3, 5 and 6 chunks of 128, which no power-of-two case has), any
expert count and top-k, per-expert gate/up and down rates, with and without a shared expert (gated
or not), both SwiGLU limits, strict or automatic geometry, 1 to 100 tokens (decode GEMV, MFMA tiles
and the two-class prefill pipeline).

Each case: routes bit-exact against the oracle's top-k, layer output within the oracle's 1e-2
row-relative tolerance, no flag raised; in strict mode every row also equals its one-row call bit
for bit. Given routes likewise, with an expert range (ids outside it inactive), experts repeated
within a token, zero weights and fp32 or fp16 weights. Captured into a hipGraph, each replay with new
inputs equals the eager call bit for bit. The single EXL3 linear likewise, over random widths (1 to 40 chunks of 128 in, 1 to 10
out), rates and row counts on both sides of its 16-row switch to the MFMA tiles."""
import numpy as np
import pytest
import torch

from oracle import coop, synth
from tests.gpu_helpers import DeviceExperts, rel_err_rows, to_dev

pytestmark = pytest.mark.gpu

TOL = 1e-2
RATES = (1.5, 2, 2.5, 3, 3.5, 4, 5)


def _draw(seed):
    rng = np.random.default_rng(9100 + seed)
    H = int(rng.choice([256, 384, 640, 768, 1024]))
    I = int(rng.choice([128, 256, 384, 640, 768]))
    E = int(rng.integers(4, 41))
    topk = int(rng.integers(1, min(8, E) + 1))
    rows = int(rng.choice([1, 2, 3, 7, 16, 17, 40, 100]))
    strict = bool(rng.random() < 0.5) and rows * topk <= 256
    return rng, dict(H=H, I=I, E=E, topk=topk, rows=rows, strict=strict,
                     has_shared=bool(rng.random() < 0.75), gated=bool(rng.random() < 0.5),
                     limit=float(rng.choice([10.0, 0.75])))


@pytest.mark.parametrize("seed", range(32))
def test_random_layer_configuration(dev, seed):
    from eva_amd import ops
    rng, c = _draw(seed)
    H, I, E, topk, rows = c["H"], c["I"], c["E"], c["topk"], c["rows"]
    rates = synth.mixed_rates(rng, E, RATES)
    drates = synth.mixed_rates(rng, E, RATES)
    experts = [synth.expert(rng, H, I, float(rates[e]), 1 / np.sqrt(H), K_down=float(drates[e])) for e in range(E)]
    sh_k, sh_kd = float(rng.choice(RATES)), float(rng.choice(RATES))
    shared = synth.expert(rng, H, I, sh_k, 1 / np.sqrt(H), K_down=sh_kd) if c["has_shared"] else None
    gate = (rng.standard_normal(H) * 0.05).astype(np.float16) if shared is not None and c["gated"] else None
    x = synth.activations_bf16(rng, rows, H)
    if rng.random() < 0.5:
        logits = synth.logits_skewed(rng, rows, E, hot=1, warm=min(3, E - 1))
    else:
        logits = synth.logits_zipf(rng, rows, E)
    ref, ridx, _, _ = coop.moe_layer(x, logits, experts, shared, topk, c["limit"], shared_gate_w=gate)

    de = DeviceExperts(experts, dev)
    kw = dict(k2_per_expert=de.k2, k2_down_per_expert=de.k2_down)
    if shared is not None:
        ds = DeviceExperts([shared], dev)
        kw.update(shared_ptrs=ds.ptrs(0), shared_bits=sh_k, shared_bits_down=sh_kd)
        if gate is not None:
            kw["shared_gate_w"] = to_dev(gate, dev)
    ws = ops.MoeWorkspace(dev, rows_max=rows, hidden=H, inter=I, topk=topk, n_local=E, has_shared=shared is not None,
                          strict_rows=rows if c["strict"] else 0)
    ws.buffer.fill_(0x5a)                        # whatever a workspace held before
    ws.clear_flags()
    xd = to_dev(x, dev).to(torch.bfloat16)
    zd = to_dev(logits, dev)

    def run(r0, T):
        sel = torch.empty(T, topk, dtype=torch.int64, device=dev)
        w = torch.empty(T, topk, dtype=torch.float32, device=dev)
        out = torch.empty(T, H, dtype=torch.float32, device=dev)
        ops.moe_forward(ws, xd[r0:r0 + T], de.table, out, limit=c["limit"], logits=zd[r0:r0 + T], sel=sel,
                        weights=w, **kw)
        torch.cuda.synchronize()
        return out.cpu().numpy(), sel.cpu().numpy()

    print("case", seed, c, flush=True)
    y, sel = run(0, rows)
    assert np.array_equal(sel, ridx)
    assert int(ws.flags().cpu()[0]) == 0
    assert rel_err_rows(y, ref) < TOL
    if c["strict"] and rows > 1:
        y1 = np.concatenate([run(r, 1)[0] for r in range(rows)])
        assert np.array_equal(y.view(np.uint32), y1.view(np.uint32))


@pytest.mark.parametrize("seed", range(16))
def test_random_given_routes(dev, seed):
    from eva_amd import ops
    rng, c = _draw(100 + seed)
    H, I, E, topk, rows = c["H"], c["I"], c["E"], c["topk"], c["rows"]
    lo = int(rng.integers(0, 20))
    hi = lo + E
    experts = [synth.expert(rng, H, I, float(rng.choice(RATES)), 1 / np.sqrt(H), K_down=float(rng.choice(RATES)))
               for _ in range(E)]
    shared = synth.expert(rng, H, I, 3.0, 1 / np.sqrt(H)) if c["has_shared"] else None
    x = synth.activations_bf16(rng, rows, H)
    sel = rng.integers(lo - 3, hi + 3, size=(rows, topk)).astype(np.int64)     # some outside the range
    if topk > 1 and rng.random() < 0.5:
        sel[:, rng.integers(0, topk)] = sel[0, 0] if lo <= sel[0, 0] < hi else lo   # one expert repeated
    w = rng.uniform(0.05, 1.0, size=(rows, topk)).astype(np.float32)
    w[rng.random((rows, topk)) < 0.15] = 0.0
    rw = w.astype(np.float16)
    xh = x.astype(np.float32).astype(np.float16)
    ref = coop.moe_routed(xh, sel, rw, dict(enumerate(experts)), c["limit"], min_expert=lo, max_expert=hi)
    if shared is not None:
        ref = ref + coop.shared_expert(xh, shared, c["limit"])
    ref = np.asarray(ref, np.float32)

    de = DeviceExperts(experts, dev)
    kw = dict(k2_per_expert=de.k2, k2_down_per_expert=de.k2_down, min_expert=lo, max_expert=hi)
    if shared is not None:
        ds = DeviceExperts([shared], dev)
        kw.update(shared_ptrs=ds.ptrs(0), shared_bits=3.0)
    ws = ops.MoeWorkspace(dev, rows_max=rows, hidden=H, inter=I, topk=topk, n_local=E, has_shared=shared is not None,
                          strict_rows=rows if c["strict"] else 0)
    ws.buffer.fill_(0xa5)
    ws.clear_flags()
    xd = to_dev(x, dev).to(torch.bfloat16)
    sd = to_dev(sel, dev)
    half = bool(rng.random() < 0.5)
    wd = to_dev(rw if half else w, dev)

    def run(r0, T):
        out = torch.empty(T, H, dtype=torch.float32, device=dev)
        wk = {"rw" if half else "weights": wd[r0:r0 + T].contiguous()}
        ops.moe_forward(ws, xd[r0:r0 + T], de.table, out, limit=c["limit"], sel=sd[r0:r0 + T].contiguous(), **wk,
                        **kw)
        torch.cuda.synchronize()
        return out.cpu().numpy()

    print("case", seed, c, dict(lo=lo, hi=hi, half=half), flush=True)
    y = run(0, rows)
    assert int(ws.flags().cpu()[0]) == 0
    assert rel_err_rows(y, ref) < TOL
    if c["strict"] and rows > 1:
        y1 = np.concatenate([run(r, 1) for r in range(rows)])
        assert np.array_equal(y.view(np.uint32), y1.view(np.uint32))


@pytest.mark.parametrize("seed", range(8))
def test_random_graph_replays(dev, seed):
    from eva_amd import ops
    rng, c = _draw(200 + seed)
    H, I, E, topk, T = c["H"], c["I"], c["E"], c["topk"], c["rows"]
    experts = [synth.expert(rng, H, I, float(rng.choice(RATES)), 1 / np.sqrt(H), K_down=float(rng.choice(RATES)))
               for _ in range(E)]
    shared = synth.expert(rng, H, I, 4.0, 1 / np.sqrt(H)) if c["has_shared"] else None
    de = DeviceExperts(experts, dev)
    kw = dict(k2_per_expert=de.k2, k2_down_per_expert=de.k2_down)
    if shared is not None:
        ds = DeviceExperts([shared], dev)
        kw.update(shared_ptrs=ds.ptrs(0), shared_bits=4.0)
    ws = ops.MoeWorkspace(dev, rows_max=T, hidden=H, inter=I, topk=topk, n_local=E, has_shared=shared is not None,
                          strict_rows=T if c["strict"] else 0)
    xs = torch.zeros(T, H, dtype=torch.bfloat16, device=dev)
    zs = torch.zeros(T, E, dtype=torch.float32, device=dev)
    sel = torch.empty(T, topk, dtype=torch.int64, device=dev)
    w = torch.empty(T, topk, dtype=torch.float32, device=dev)
    out = torch.empty(T, H, dtype=torch.float32, device=dev)

    def fwd():
        ops.moe_forward(ws, xs, de.table, out, limit=c["limit"], logits=zs, sel=sel, weights=w, **kw)

    print("case", seed, c, flush=True)
    fwd()                                        # outside capture first (a call of more than 16 tokens makes its side stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fwd()
    torch.cuda.synchronize()
    for rep in range(3):
        x = synth.activations_bf16(rng, T, H)
        z = synth.logits_zipf(rng, T, E)
        xs.copy_(to_dev(x, dev).to(torch.bfloat16))
        zs.copy_(to_dev(z, dev))
        graph.replay()
        torch.cuda.synchronize()
        y_graph, idx_graph = out.clone(), sel.clone()
        fwd()                                    # eager on the same inputs
        torch.cuda.synchronize()
        assert torch.equal(idx_graph, sel), rep
        assert torch.equal(y_graph, out), rep
        ref, ridx, _, _ = coop.moe_layer(x, z, experts, shared, topk, c["limit"])
        assert np.array_equal(idx_graph.cpu().numpy(), ridx)
        assert rel_err_rows(y_graph.cpu().numpy(), ref) < TOL


@pytest.mark.parametrize("seed", range(24))
def test_random_linear_configuration(dev, seed):
    from eva_amd import ops
    rng = np.random.default_rng(9300 + seed)
    n_in = 128 * int(rng.choice([1, 3, 5, 9, 16, 40]))
    n_out = 128 * int(rng.choice([1, 3, 5, 7, 10]))
    rows = int(rng.choice([1, 2, 3, 9, 16, 17, 50]))
    K = float(rng.choice(RATES))
    print("case", seed, dict(n_in=n_in, n_out=n_out, rows=rows, K=K), flush=True)
    tr, suh, svh = synth.projection(rng, n_in, n_out, K, svh_scale=1 / np.sqrt(n_in))
    x = rng.standard_normal((rows, n_in)).astype(np.float16)
    ws = torch.full((ops.lib().evamx_exl3_linear_workspace_bytes(rows, n_in, n_out),), 0x5a, dtype=torch.uint8,
                    device=dev)
    y = ops.exl3_linear(to_dev(x, dev), to_dev(tr, dev), to_dev(suh, dev), to_dev(svh, dev), K, workspace=ws)
    ref = coop.exl3_linear(x, tr, suh, svh, K)
    assert rel_err_rows(y.cpu().numpy().astype(np.float32), ref.astype(np.float32)) < TOL
