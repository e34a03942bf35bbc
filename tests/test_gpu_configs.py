"""Parity at the BASELINE configurations' shapes (configs[0..4]) on the GPU.

- config 1: the single EXL3 linear 2048 -> 7168 at 4 bpw, 1 token: decoded weights bit-exact,
  output within tolerance;
- config 3 (T=16, per-token-bias routing) is covered at the DSv3 shape in test_gpu_parity;
- config 4: 512-token prefill with Zipf routing and per-expert rates {2,3,4,5}: the oracle on a
  reduced width, and at the full DSv3 width a batch-invariance property (each row of the
  512-row call equals the same row run alone) plus the oracle on two rows;
- config 5: stacked layers at 2.5 bpw with the fused bf16 residual, against the oracle's stack
  (3 reduced-width layers eager, and 3 DSv3-width layers captured as one hipGraph).
Bars: indices bit-exact; outputs within max row-relative error 1e-2.
"""
import numpy as np
import pytest
import torch

from oracle import coop, exl3, synth
from tests.gpu_helpers import DeviceExperts, clamp_variants, rel_err_rows, to_dev

pytestmark = pytest.mark.gpu
TOL = 1e-2
CLIP = 0.75          # SwiGLU limit that clips ~12% of SiLU(G) and ~45% of U at these scales


def test_config1_linear(dev):
    from eva_amd import ops
    rng = np.random.default_rng(101)
    tr, suh, svh = synth.projection(rng, 2048, 7168, 4)
    x = synth.activations_bf16(rng, 1, 2048).astype(np.float16)
    dtr = to_dev(tr, dev)
    w = ops.exl3_dequant(dtr, 4).cpu().numpy()
    W = coop.dequant_fast(tr, 4)
    assert np.array_equal(w.view(np.uint16), W.view(np.uint16))
    y = ops.exl3_linear(to_dev(x, dev), dtr, to_dev(suh, dev), to_dev(svh, dev), 4).cpu().numpy()
    ref = coop.exl3_linear(x, tr, suh, svh, 4, W=W)
    assert rel_err_rows(y.astype(np.float32), ref.astype(np.float32)) < TOL


def test_config1_linear_128_rows(dev):
    """configs[0]'s layer at 128 rows (the MFMA path of the linear) against the oracle."""
    from eva_amd import ops
    rng = np.random.default_rng(111)
    tr, suh, svh = synth.projection(rng, 2048, 7168, 4)
    x = synth.activations_bf16(rng, 128, 2048).astype(np.float16)
    y = ops.exl3_linear(to_dev(x, dev), to_dev(tr, dev), to_dev(suh, dev), to_dev(svh, dev), 4).cpu().numpy()
    ref = coop.exl3_linear(x, tr, suh, svh, 4)
    assert rel_err_rows(y.astype(np.float32), ref.astype(np.float32)) < TOL


def _moe(ops, dev, H, I, E, topk, rows, experts_dev, k2, x, logits, shared_dev=None, shared_bits=None, limit=10.0):
    ws = ops.MoeWorkspace(dev, rows_max=rows, hidden=H, inter=I, topk=topk, n_local=E,
                          has_shared=shared_dev is not None)
    sel = torch.empty(rows, topk, dtype=torch.int64, device=dev)
    w = torch.empty(rows, topk, dtype=torch.float32, device=dev)
    out = torch.empty(rows, H, dtype=torch.float32, device=dev)
    ops.moe_forward(ws, x, experts_dev, out, limit=limit, k2_per_expert=k2, logits=logits, sel=sel, weights=w,
                    shared_ptrs=shared_dev, shared_bits=shared_bits)
    torch.cuda.synchronize()
    assert int(ws.flags().cpu()[0]) == 0
    return out, sel


@pytest.mark.parametrize("limit", [10.0, CLIP])
def test_config4_prefill_reduced(dev, limit):
    """512 tokens, Zipf routing, rates {2,3,4,5} through the 16- and 64-row MFMA kernels; at CLIP
    the SwiGLU limit clips in the routed (after SiLU) and the shared (before SiLU) expert, and
    the result must be far from the layer with either clamp order swapped or no clamp."""
    from eva_amd import ops
    H, I, E, topk, T = 1024, 256, 64, 8, 512
    rng = np.random.default_rng(104)
    rates = synth.mixed_rates(rng, E)
    experts = [synth.expert(rng, H, I, float(r), 1 / np.sqrt(H)) for r in rates]
    shared = synth.expert(rng, H, I, 4, 1 / np.sqrt(H))
    x = synth.activations_bf16(rng, T, H)
    logits = synth.logits_zipf(rng, T, E)
    compute = lambda: coop.moe_layer(x, logits, experts, shared, topk, limit)[0]
    variants = clamp_variants(compute) if limit == CLIP else {"ref": compute()}
    ridx, _ = coop.route(logits, topk)
    de, ds = DeviceExperts(experts, dev), DeviceExperts([shared], dev)
    out, sel = _moe(ops, dev, H, I, E, topk, T, de.table, de.k2, to_dev(x, dev).to(torch.bfloat16),
                    to_dev(logits, dev), ds.ptrs(0), 4.0, limit=limit)
    assert np.array_equal(sel.cpu().numpy(), ridx)
    y = out.cpu().numpy()
    assert rel_err_rows(y, variants["ref"]) < TOL
    if limit == CLIP:
        for name in ("routed_swapped", "shared_swapped", "unclamped"):
            assert rel_err_rows(variants[name], variants["ref"]) > 5 * TOL, name
            assert rel_err_rows(y, variants[name]) > 2 * TOL, name


@pytest.mark.parametrize("T,zipf", [(512, True), (40, False)])
def test_prefill_forms_bit_identical(dev, T, zipf):
    """The MFMA stages' launch forms accumulate every column over the same k-steps in the same
    order, so the layer's output is bit-identical across them: the default (tiles of at most 16
    rows in the 16-row kernel on a side stream, concurrently with the larger ones) and
    EVAMX_PREFILL_CONCURRENT=0 (one kernel on the caller's stream); and within the tolerance of
    the oracle, with the SwiGLU limit clipping. 512 Zipf tokens give tiles of 1-4
    row blocks; 40 tokens give automatic k-splits."""
    import os
    from eva_amd import ops
    H, I, E, topk = 1024, 256, 64, 8
    rng = np.random.default_rng(105 + T)
    rates = synth.mixed_rates(rng, E)
    experts = [synth.expert(rng, H, I, float(r), 1 / np.sqrt(H)) for r in rates]
    shared = synth.expert(rng, H, I, 4, 1 / np.sqrt(H))
    x = synth.activations_bf16(rng, T, H)
    logits = synth.logits_zipf(rng, T, E) if zipf else synth.logits_plain(rng, T, E)
    de, ds = DeviceExperts(experts, dev), DeviceExperts([shared], dev)
    outs = []
    for env in ({}, {"EVAMX_PREFILL_CONCURRENT": "0"}):
        os.environ.update(env)
        try:
            out, _ = _moe(ops, dev, H, I, E, topk, T, de.table, de.k2, to_dev(x, dev).to(torch.bfloat16),
                          to_dev(logits, dev), ds.ptrs(0), 4.0, limit=CLIP)
        finally:
            for key in env:
                os.environ.pop(key, None)
        outs.append(out.cpu().numpy())
    assert np.array_equal(outs[0], outs[1])
    ref = coop.moe_layer(x, logits, experts, shared, topk, CLIP)[0]
    assert rel_err_rows(outs[1], ref) < TOL


@pytest.mark.parametrize("T,E,shared", [(24, 64, False), (64, 4, True)])
def test_prefill_one_size_class_empty(dev, T, E, shared):
    """Calls of more than 16 tokens whose tiles fall in one size class only: 24 tokens over 64
    experts with no shared expert (every tile at most 16 rows: the 64-row kernels and the larger
    class's activation have no work), 64 tokens over 4 experts and the shared one (every tile
    64 rows: the side stream's kernels have none). Bit-identical to the single-stream form and
    within the tolerance of the oracle."""
    import os
    from eva_amd import ops
    H, I, topk = 512, 256, 2
    rng = np.random.default_rng(300 + T)
    experts = [synth.expert(rng, H, I, 4, 1 / np.sqrt(H)) for _ in range(E)]
    sh = synth.expert(rng, H, I, 4, 1 / np.sqrt(H)) if shared else None
    x = synth.activations_bf16(rng, T, H)
    logits = synth.logits_plain(rng, T, E)
    de = DeviceExperts(experts, dev)
    ds = DeviceExperts([sh], dev) if shared else None
    outs = []
    for env in ({}, {"EVAMX_PREFILL_CONCURRENT": "0"}):
        os.environ.update(env)
        try:
            out, sel = _moe(ops, dev, H, I, E, topk, T, de.table, de.k2, to_dev(x, dev).to(torch.bfloat16),
                            to_dev(logits, dev), ds.ptrs(0) if shared else None, 4.0 if shared else None, limit=CLIP)
        finally:
            for key in env:
                os.environ.pop(key, None)
        outs.append(out.cpu().numpy())
    assert np.array_equal(outs[0], outs[1])
    ref = coop.moe_layer(x, logits, experts, sh, topk, CLIP)[0]
    assert rel_err_rows(outs[0], ref) < TOL


class _DeviceRandomExperts:
    """E experts at per-expert rates, drawn on the device (seeded), with a [9, E] pointer table."""

    def __init__(self, dev, H, I, rates, seed):
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        self.parts = []
        rows = [[0] * len(rates) for _ in range(9)]
        for e, K in enumerate(rates):
            ps = []
            for p, (n_in, n_out) in enumerate(((H, I), (H, I), (I, H))):
                tr = torch.empty(n_in // 16, n_out // 16, exl3.tile_u16(K), dtype=torch.int16, device=dev)
                tr.random_(-32768, 32768, generator=g)
                suh = (torch.randint(0, 2, (n_in,), generator=g, device=dev) * 2 - 1).half()
                mag = torch.rand(n_out, generator=g, device=dev) + 0.5
                svh = ((torch.randint(0, 2, (n_out,), generator=g, device=dev) * 2 - 1) * mag / H ** 0.5).half()
                ps.append((tr, suh, svh))
                for j, t in enumerate((tr, suh, svh)):
                    rows[3 * p + j][e] = t.data_ptr()
            self.parts.append(ps)
        self.table = torch.tensor(rows, dtype=torch.int64, device=dev)
        self.k2 = torch.tensor([int(round(2 * K)) for K in rates], dtype=torch.uint8, device=dev)
        self.rates = rates

    def oracle_expert(self, e):
        ps = [tuple(t.cpu().numpy() for t in part) for part in self.parts[e]]
        return coop.ExpertWeights(*ps, K=float(self.rates[e]))


def test_config4_full_width_batch_invariance(dev):
    from eva_amd import ops
    H, I, E, topk, T = 7168, 2048, 256, 8, 512
    rng = np.random.default_rng(204)
    rates = [float(r) for r in synth.mixed_rates(rng, E)]
    de = _DeviceRandomExperts(dev, H, I, rates + [4.0], seed=2040)
    table = de.table[:, :E].contiguous()
    k2 = de.k2[:E].contiguous()
    shared_ptrs = [int(v) for v in de.table[:, E].cpu()]
    x = to_dev(synth.activations_bf16(rng, T, H), dev).to(torch.bfloat16)
    logits_np = synth.logits_zipf(rng, T, E)
    logits = to_dev(logits_np, dev)
    out, sel = _moe(ops, dev, H, I, E, topk, T, table, k2, x, logits, shared_ptrs, 4.0)
    ridx, _ = coop.route(logits_np, topk)
    assert np.array_equal(sel.cpu().numpy(), ridx)
    y = out.cpu().numpy()
    rows = [0, 1, 77, 300, 511]
    for r in rows:                                         # each row alone gives the same row
        o1, s1 = _moe(ops, dev, H, I, E, topk, 1, table, k2, x[r:r + 1], logits[r:r + 1], shared_ptrs, 4.0)
        assert np.array_equal(s1.cpu().numpy()[0], ridx[r])
        assert rel_err_rows(o1.cpu().numpy(), y[r:r + 1]) < 2e-3, r
    for r in rows[:2]:                                     # and the oracle on two rows
        experts = {int(e): de.oracle_expert(int(e)) for e in ridx[r]}
        shared = de.oracle_expert(E)
        ref, _, _, _ = coop.moe_layer(x[r:r + 1].float().cpu().numpy(), logits_np[r:r + 1], experts, shared, topk, 10.0)
        assert rel_err_rows(y[r:r + 1], ref) < TOL, r


def test_config5_stack_residual(dev):
    from eva_amd import ops
    H, I, E, topk, T, L, K = 512, 256, 16, 4, 8, 3, 2.5
    rng = np.random.default_rng(105)
    layers = []
    for _ in range(L):
        layers.append(([synth.expert(rng, H, I, K, 1 / np.sqrt(H)) for _ in range(E)],
                       synth.expert(rng, H, I, K, 1 / np.sqrt(H))))
    h0 = synth.activations_bf16(rng, T, H)
    logits = [synth.logits_plain(rng, T, E) for _ in range(L)]
    ref = coop.layer_stack(h0, logits, layers, topk, 10.0)
    dev_layers = [(DeviceExperts(ex, dev), DeviceExperts([sh], dev)) for ex, sh in layers]
    ws = ops.MoeWorkspace(dev, rows_max=T, hidden=H, inter=I, topk=topk, n_local=E, has_shared=True)
    h = to_dev(h0, dev).to(torch.bfloat16)
    sel = torch.empty(T, topk, dtype=torch.int64, device=dev)
    w = torch.empty(T, topk, dtype=torch.float32, device=dev)
    for l, (de, ds) in enumerate(dev_layers):
        ops.moe_forward(ws, h, de.table, None, limit=10.0, bits=K, logits=to_dev(logits[l], dev), sel=sel, weights=w,
                        shared_ptrs=ds.ptrs(0), shared_bits=K, residual=h)
    torch.cuda.synchronize()
    got = h.float().cpu().numpy()
    assert rel_err_rows(got, ref) < TOL
    # the layers' contribution, allowing one bf16 half-ulp per residual rounding per layer
    bound = L * np.maximum(np.abs(ref), np.abs(got)) * 2.0 ** -8 + TOL * np.abs(ref - h0).max()
    assert np.all(np.abs(got - ref) <= bound)


def test_config5_dsv3_width_layers_in_one_graph(dev):
    """configs[4] at its real width: 3 DSv3-shape layers (H=7168, I=2048, 256 routed + 1 shared,
    top-8) at 2.5 bpw, 8 tokens, independent seeded routing per layer, each layer adding its
    output into the bf16 residual stream (model.py:498-499), the whole step captured as ONE
    hipGraph. Every replay (with eager work in between) must give the same bits as the eager
    step, and the stream must match the oracle's layer_stack on the touched experts."""
    from eva_amd import ops
    H, I, E, topk, T, L, K, limit = 7168, 2048, 256, 8, 8, 3, 2.5, 10.0
    rng = np.random.default_rng(505)
    logits = [synth.logits_skewed(rng, T, E, hot=2, warm=6) for _ in range(L)]
    h0 = synth.activations_bf16(rng, T, H)
    dummy = synth.expert(rng, H, I, K, 1 / np.sqrt(H))
    layers, tables, shared_ptrs, keep = [], [], [], []
    for l in range(L):
        used = sorted(set(int(v) for v in coop.route(logits[l], topk)[0].reshape(-1)))
        experts = {e: synth.expert(rng, H, I, K, 1 / np.sqrt(H)) for e in used}
        shared = synth.expert(rng, H, I, K, 1 / np.sqrt(H))
        layers.append((experts, shared))
        de = DeviceExperts([experts[e] for e in used] + [dummy], dev)
        host = de.table.cpu()
        cols = {e: i for i, e in enumerate(used)}
        tables.append(torch.stack([host[:, cols.get(e, len(used))] for e in range(E)], dim=1).contiguous().to(dev))
        ds = DeviceExperts([shared], dev)
        shared_ptrs.append(ds.ptrs(0))
        keep += [de, ds]
    ref = coop.layer_stack(h0, logits, layers, topk, limit)

    ws = ops.MoeWorkspace(dev, rows_max=T, hidden=H, inter=I, topk=topk, n_local=E, has_shared=True)
    h_in = to_dev(h0, dev).to(torch.bfloat16)
    h = torch.empty_like(h_in)
    z = [to_dev(v, dev) for v in logits]
    sel = torch.empty(L, T, topk, dtype=torch.int64, device=dev)
    w = torch.empty(L, T, topk, dtype=torch.float32, device=dev)

    def step():
        h.copy_(h_in)
        for l in range(L):
            ops.moe_forward(ws, h, tables[l], None, limit=limit, bits=K, logits=z[l], sel=sel[l], weights=w[l],
                            shared_ptrs=shared_ptrs[l], shared_bits=K, residual=h)

    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        step()
    torch.cuda.synchronize()
    eager = h.clone()
    for l in range(L):
        assert np.array_equal(sel[l].cpu().numpy(), coop.route(logits[l], topk)[0])
    assert rel_err_rows(eager.float().cpu().numpy(), ref) < TOL
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            step()
    for i in range(3):
        h.fill_(0)                                         # eager work between the replays
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(h, eager), i
