"""One-row calls route inside the gate/up launch (no prepare launch): every routed wave routes the
token itself and one extra workgroup publishes the routes, run table and unit/slot records. These
cases check that path's own edges against the CPU oracle: the EP filter and zero weights leaving
slots inactive (exl3_moe_coop_kernel.cuh:208-223), a token with no active slot (shared term only,
or zeros), an out-of-range expert (flagged and dropped), the published run table
(moe_coop3072.py:86-106), and hipGraph replays of the routed call."""
import numpy as np
import pytest
import torch

from oracle import coop, synth
from tests.gpu_helpers import DeviceExperts, rel_err_rows, to_dev

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _experts(rng, H, I, E, K):
    return [synth.expert(rng, H, I, K, 1 / np.sqrt(H)) for _ in range(E)]


@pytest.mark.parametrize("shared", [False, True])
def test_one_row_expert_range_and_zero_weights(dev, shared):
    """Given routes at one row: picks outside [lo, hi) and a zero weight are inactive slots (their
    waves exit); the rest match the oracle, the run table matches the reference's."""
    from eva_amd import ops
    H, I, k = 256, 128, 8
    lo, hi = 4, 12
    rng = np.random.default_rng(41)
    ex = _experts(rng, H, I, hi - lo, 3)
    sh = synth.expert(rng, H, I, 3, 1 / np.sqrt(H))
    x = rng.standard_normal((1, H)).astype(np.float16)
    sel = np.array([[5, 1, 11, 13, 4, 7, 0, 9]], dtype=np.int64)      # 1, 13, 0 outside [4, 12)
    rw = rng.uniform(0.1, 1, size=(1, k)).astype(np.float16)
    rw[0, 5] = 0                                                      # expert 7: zero weight
    ref = coop.moe_routed(x, sel, rw, ex, 10.0, min_expert=lo, max_expert=hi)
    if shared:
        ref = ref + coop.shared_expert(x, sh, 10.0)
    de, ds = DeviceExperts(ex, dev), DeviceExperts([sh], dev)
    ws = ops.MoeWorkspace(dev, rows_max=1, hidden=H, inter=I, topk=k, n_local=hi - lo, has_shared=shared)
    ws.buffer.fill_(0x7f)                                             # no stale records or partials
    ws.clear_flags()
    out = torch.full((1, H), float("nan"), dtype=torch.float32, device=dev)
    ops.moe_forward(ws, to_dev(x, dev), de.table, out, limit=10.0, bits=3, sel=to_dev(sel, dev), rw=to_dev(rw, dev),
                    min_expert=lo, max_expert=hi, shared_ptrs=ds.ptrs(0) if shared else None,
                    shared_bits=3 if shared else None)
    torch.cuda.synchronize()
    assert int(ws.flags().cpu()[0]) == 0                              # range misses are not errors
    assert rel_err_rows(out.cpu().numpy(), ref) < TOL
    ok, _ = coop.slot_active(sel, rw, lo, hi)
    assert ok.sum() == 4
    want = coop.reference_table(np.where(ok, sel - lo, 0), np.where(ok, rw, 0), capacity=1)
    assert np.array_equal(ws.runs().cpu().numpy(), want)


@pytest.mark.parametrize("shared", [False, True])
def test_one_row_no_active_slot(dev, shared):
    """Every weight zero: the routed part is empty; the output is the shared term, or zeros."""
    from eva_amd import ops
    H, I, E, k = 256, 128, 6, 4
    rng = np.random.default_rng(42)
    ex = _experts(rng, H, I, E, 4)
    sh = synth.expert(rng, H, I, 4, 1 / np.sqrt(H))
    x = rng.standard_normal((1, H)).astype(np.float16)
    sel = np.array([[0, 1, 2, 3]], dtype=np.int64)
    rw = np.zeros((1, k), dtype=np.float16)
    de, ds = DeviceExperts(ex, dev), DeviceExperts([sh], dev)
    ws = ops.MoeWorkspace(dev, rows_max=1, hidden=H, inter=I, topk=k, n_local=E, has_shared=shared)
    out = torch.full((1, H), float("nan"), dtype=torch.float32, device=dev)
    ops.moe_forward(ws, to_dev(x, dev), de.table, out, limit=10.0, bits=4, sel=to_dev(sel, dev), rw=to_dev(rw, dev),
                    shared_ptrs=ds.ptrs(0) if shared else None, shared_bits=4 if shared else None)
    torch.cuda.synchronize()
    y = out.cpu().numpy()
    if shared:
        assert rel_err_rows(y, coop.shared_expert(x, sh, 10.0)) < TOL
    else:
        assert np.all(y == 0)
    assert np.all(ws.runs().cpu().numpy() == 0)


def test_one_row_out_of_range_expert_sets_flag(dev):
    from eva_amd import ops
    H, I, E, k = 256, 128, 8, 4
    rng = np.random.default_rng(43)
    ex = _experts(rng, H, I, E, 4)
    de = DeviceExperts(ex, dev)
    ws = ops.MoeWorkspace(dev, rows_max=1, hidden=H, inter=I, topk=k, n_local=E, has_shared=False)
    x = rng.standard_normal((1, H)).astype(np.float16)
    sel = np.array([[3, 99, 5, 0]], dtype=np.int64)                  # 99 is outside the table
    rw = np.array([[0.25, 0.5, 0.125, 0.5]], dtype=np.float16)
    out = torch.empty(1, H, dtype=torch.float32, device=dev)
    ops.moe_forward(ws, to_dev(x, dev), de.table, out, limit=0.0, bits=4, sel=to_dev(sel, dev), rw=to_dev(rw, dev))
    torch.cuda.synchronize()
    assert int(ws.flags().cpu()[0]) & 1
    rw2 = rw.copy()
    rw2[0, 1] = 0                                                     # the flagged slot is dropped
    ref = coop.moe_routed(x, np.where(sel < E, sel, 0), rw2, ex, 0.0)
    assert rel_err_rows(out.cpu().numpy(), ref) < TOL


def test_one_row_graph_replays(dev):
    """A captured one-row forward routed from logits, replayed with new inputs: routes, weights
    and output of every replay equal the eager call's and the oracle's; the run table too."""
    from eva_amd import ops
    H, I, E, k = 256, 128, 16, 4
    rng = np.random.default_rng(44)
    ex = _experts(rng, H, I, E, 4)
    sh = synth.expert(rng, H, I, 4, 1 / np.sqrt(H))
    de, ds = DeviceExperts(ex, dev), DeviceExperts([sh], dev)
    ws = ops.MoeWorkspace(dev, rows_max=1, hidden=H, inter=I, topk=k, n_local=E, has_shared=True)
    xs = torch.zeros(1, H, dtype=torch.bfloat16, device=dev)
    zs = torch.zeros(1, E, dtype=torch.float32, device=dev)
    sel = torch.empty(1, k, dtype=torch.int64, device=dev)
    w = torch.empty(1, k, dtype=torch.float32, device=dev)
    out = torch.empty(1, H, dtype=torch.float32, device=dev)

    def fwd():
        ops.moe_forward(ws, xs, de.table, out, limit=10.0, bits=4, logits=zs, sel=sel, weights=w,
                        shared_ptrs=ds.ptrs(0), shared_bits=4)

    fwd()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fwd()
    torch.cuda.synchronize()
    for rep in range(4):
        x = synth.activations_bf16(rng, 1, H)
        z = synth.logits_plain(rng, 1, E)
        xs.copy_(to_dev(x, dev).to(torch.bfloat16))
        zs.copy_(to_dev(z, dev))
        graph.replay()
        torch.cuda.synchronize()
        y_graph, idx_graph, w_graph = out.clone(), sel.clone(), w.clone()
        runs_graph = ws.runs().clone()
        fwd()                                                         # eager on the same inputs
        torch.cuda.synchronize()
        assert torch.equal(idx_graph, sel) and torch.equal(w_graph, w), rep
        assert torch.equal(y_graph, out), rep
        ref, ridx, rw32, rrw = coop.moe_layer(x, z, ex, sh, k, 10.0)
        assert np.array_equal(idx_graph.cpu().numpy(), ridx)
        assert np.array_equal(w_graph.cpu().numpy(), rw32)
        assert np.array_equal(runs_graph.cpu().numpy(), coop.reference_table(ridx, rrw, capacity=1))
        assert rel_err_rows(y_graph.cpu().numpy(), ref) < TOL



@pytest.mark.parametrize("E,k,score,bias", [(384, 16, "sigmoid", False), (384, 8, "sqrt_softplus", True),
                                            (64, 32, "sigmoid", True)])
def test_one_row_routing_variants(dev, E, k, score, bias):
    """Routing inside the gate/up launch beyond the DSv3 defaults: more than 256 experts (eight
    keys per lane), top-16 and top-32 (the shared expert's unit after 32 routed ones), the
    sqrt-softplus score and a selection bias (model.py:404-416). Indices and weights are the
    oracle's bit for bit, the run table is the reference's, the output within the tolerance."""
    from eva_amd import ops
    H, I = 256, 128
    rng = np.random.default_rng(46 + k)
    ex = _experts(rng, H, I, E, 2)
    sh = synth.expert(rng, H, I, 2, 1 / np.sqrt(H))
    de, ds = DeviceExperts(ex, dev), DeviceExperts([sh], dev)
    x = synth.activations_bf16(rng, 1, H)
    z = synth.logits_plain(rng, 1, E)
    b = (rng.standard_normal(E) * 0.5).astype(np.float32) if bias else None
    ws = ops.MoeWorkspace(dev, rows_max=1, hidden=H, inter=I, topk=k, n_local=E, has_shared=True)
    sel = torch.empty(1, k, dtype=torch.int64, device=dev)
    w = torch.empty(1, k, dtype=torch.float32, device=dev)
    out = torch.empty(1, H, dtype=torch.float32, device=dev)
    ops.moe_forward(ws, to_dev(x, dev).to(torch.bfloat16), de.table, out, limit=10.0, bits=2, logits=to_dev(z, dev),
                    sel=sel, weights=w, shared_ptrs=ds.ptrs(0), shared_bits=2, score_fn=score,
                    sel_bias=None if b is None else to_dev(b, dev), route_scale=2.5)
    torch.cuda.synchronize()
    ref, ridx, rw32, rrw = coop.moe_layer(x, z, ex, sh, k, 10.0, score_fn=score, sel_bias=b, route_scale=2.5)
    assert np.array_equal(sel.cpu().numpy(), ridx)
    assert np.array_equal(w.cpu().numpy(), rw32)
    assert int(ws.flags().cpu()[0]) == 0
    assert np.array_equal(ws.runs().cpu().numpy(), coop.reference_table(ridx, rrw, capacity=1))
    assert rel_err_rows(out.cpu().numpy(), ref) < TOL
