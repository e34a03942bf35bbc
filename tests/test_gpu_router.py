"""Router front on the GPU: logits computed from the fp32 gate weight inside the MoE forward.

Block.route (model.py:404-416) computes ``stable_linear(x.float(), gate_w)`` and routes on it;
``moe_forward(gate_w=...)`` does both on the device. The logits are fp32 dot products of length
H, so they are held to the textbook accumulation bound against float64 (not to one summation
order); everything after them is held bit-exact: the routes must be the oracle's routes of the
very logits the kernel wrote, and the layer output the oracle's layer on those logits. Each
row's logits must not depend on the other rows of the batch (the per-row reduction of
stable_linear, model.py:158-165).
"""
import numpy as np
import pytest
import torch

from oracle import coop, synth
from tests.gpu_helpers import DeviceExperts, rel_err_rows, to_dev

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _ops():
    from eva_amd import ops
    return ops


def _gate(rng, E, H):
    return (rng.standard_normal((E, H)) / np.sqrt(H)).astype(np.float32)


def _check_logits(z, x, gate_w):
    """|z - x.w| <= gamma_n * sum|x||w| with n = H/64 + 6 + 2 (per-lane chain, butterfly, slack)."""
    xd, wd = x.astype(np.float64), gate_w.astype(np.float64)
    exact = xd @ wd.T
    n = x.shape[1] // 64 + 8
    bound = n * 2.0 ** -24 * (np.abs(xd) @ np.abs(wd).T)
    assert np.all(np.abs(z.astype(np.float64) - exact) <= bound)


@pytest.mark.parametrize("rows", [1, 5, 40])
@pytest.mark.parametrize("score_fn,biased", [("sigmoid", False), ("sqrt_softplus", True)])
def test_moe_layer_from_gate_weight(dev, rows, score_fn, biased):
    ops = _ops()
    H, I, E, topk, limit, K = 512, 256, 24, 4, 10.0, 4
    rng = np.random.default_rng(7 * rows + biased)
    experts = [synth.expert(rng, H, I, K, 1 / np.sqrt(H)) for _ in range(E)]
    shared = synth.expert(rng, H, I, K, 1 / np.sqrt(H))
    x = synth.activations_bf16(rng, rows, H)
    gate_w = _gate(rng, E, H)
    bias = (0.1 * rng.standard_normal(E)).astype(np.float32) if biased else None

    de = DeviceExperts(experts, dev)
    ds = DeviceExperts([shared], dev)
    ws = ops.MoeWorkspace(dev, rows_max=max(rows, 16), hidden=H, inter=I, topk=topk, n_local=E, has_shared=True)
    xt = to_dev(x, dev).to(torch.bfloat16)
    sel = torch.empty(rows, topk, dtype=torch.int64, device=dev)
    w = torch.empty(rows, topk, dtype=torch.float32, device=dev)
    out = torch.empty(rows, H, dtype=torch.float32, device=dev)
    ops.moe_forward(ws, xt, de.table, out, limit=limit, bits=K, gate_w=to_dev(gate_w, dev), sel=sel, weights=w,
                    score_fn=score_fn, sel_bias=None if bias is None else to_dev(bias, dev),
                    shared_ptrs=ds.ptrs(0), shared_bits=K)
    torch.cuda.synchronize()
    assert int(ws.flags().cpu()[0]) == 0
    z = ws.logits(rows, E).cpu().numpy().copy()
    xf = xt.float().cpu().numpy()
    _check_logits(z, xf, gate_w)

    ridx, rwt = coop.route(z, topk, score_fn, bias)
    assert np.array_equal(sel.cpu().numpy(), ridx)
    assert np.array_equal(w.cpu().numpy(), rwt)
    ref, _, _, _ = coop.moe_layer(x, z, experts, shared, topk, limit, score_fn=score_fn, sel_bias=bias)
    assert rel_err_rows(out.cpu().numpy(), ref) < TOL


def test_gate_logits_dsv3_shape_and_batch_invariance(dev):
    """H=7168, 256 experts: logits within the bound, and each row's logits bit-identical whether
    it runs alone or inside a 40-row batch (decode and prefill groupings differ)."""
    ops = _ops()
    H, I, E, topk, K = 7168, 2048, 256, 8, 4
    rng = np.random.default_rng(11)
    rows = 40
    x = synth.activations_bf16(rng, rows, H)
    gate_w = to_dev(_gate(rng, E, H), dev)
    dummy = DeviceExperts([synth.expert(rng, H, I, K, 1 / np.sqrt(H))], dev)
    table = dummy.table[:, :1].expand(9, E).contiguous()
    xt = to_dev(x, dev).to(torch.bfloat16)

    def logits_of(xs):
        n = xs.shape[0]
        ws = ops.MoeWorkspace(dev, rows_max=n, hidden=H, inter=I, topk=topk, n_local=E, has_shared=False)
        sel = torch.empty(n, topk, dtype=torch.int64, device=dev)
        w = torch.empty(n, topk, dtype=torch.float32, device=dev)
        out = torch.empty(n, H, dtype=torch.float32, device=dev)
        ops.moe_forward(ws, xs, table, out, limit=10.0, bits=K, gate_w=gate_w, sel=sel, weights=w)
        torch.cuda.synchronize()
        assert int(ws.flags().cpu()[0]) == 0
        assert torch.isfinite(out).all()
        z = ws.logits(n, E).cpu().numpy().copy()
        ridx, rwt = coop.route(z, topk)
        assert np.array_equal(sel.cpu().numpy(), ridx)
        assert np.array_equal(w.cpu().numpy(), rwt)
        return z

    z_all = logits_of(xt)
    _check_logits(z_all, xt.float().cpu().numpy(), gate_w.cpu().numpy())
    for r in (0, 7, 8, 39):
        assert np.array_equal(logits_of(xt[r:r + 1].contiguous())[0].view(np.uint32), z_all[r].view(np.uint32))
    assert np.array_equal(logits_of(xt[3:19].contiguous()).view(np.uint32), z_all[3:19].view(np.uint32))


def test_gate_weight_path_is_graph_capturable(dev):
    """The gate kernel inside a captured forward: new activations copied in between replays,
    every replay equal to the eager forward on the same inputs."""
    ops = _ops()
    H, I, E, topk, K, rows = 512, 256, 24, 4, 3, 3
    rng = np.random.default_rng(5)
    experts = [synth.expert(rng, H, I, K, 1 / np.sqrt(H)) for _ in range(E)]
    de = DeviceExperts(experts, dev)
    gate_w = to_dev(_gate(rng, E, H), dev)
    ws = ops.MoeWorkspace(dev, rows_max=rows, hidden=H, inter=I, topk=topk, n_local=E, has_shared=False)
    xs = torch.zeros(rows, H, dtype=torch.bfloat16, device=dev)
    sel = torch.empty(rows, topk, dtype=torch.int64, device=dev)
    w = torch.empty(rows, topk, dtype=torch.float32, device=dev)
    out = torch.empty(rows, H, dtype=torch.float32, device=dev)

    def fwd():
        ops.moe_forward(ws, xs, de.table, out, limit=10.0, bits=K, gate_w=gate_w, sel=sel, weights=w)

    fwd()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fwd()
    torch.cuda.synchronize()
    for rep in range(3):
        xs.copy_(to_dev(synth.activations_bf16(rng, rows, H), dev).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        y_graph, idx_graph, w_graph = out.clone(), sel.clone(), w.clone()
        fwd()
        torch.cuda.synchronize()
        assert torch.equal(idx_graph, sel) and torch.equal(w_graph, w) and torch.equal(y_graph, out), rep


@pytest.mark.parametrize("rows", [1, 7, 33])
def test_block_route_mirror(dev, rows):
    """ops.route (Block.route, model.py:404-416): standalone logits within the bound and equal to the
    fused forward's; sqrt-softplus scores with gate_b, gate_b_vl on the image rows, route_scale 2.5;
    indices and weights bit-exact against the oracle router on those logits."""
    ops = _ops()
    H, E, topk = 7168, 256, 8
    rng = np.random.default_rng(100 + rows)
    x = synth.activations_bf16(rng, rows, H)
    gate_w = _gate(rng, E, H)
    gate_b = (0.05 * rng.standard_normal(E)).astype(np.float32)
    gate_b_vl = (0.05 * rng.standard_normal(E)).astype(np.float32)
    mask = rng.integers(0, 2, size=rows).astype(bool)
    xt = to_dev(x, dev).to(torch.bfloat16)
    z = ops.router_logits(xt, to_dev(gate_w, dev))
    w, idx = ops.route(xt, to_dev(gate_w, dev), to_dev(gate_b, dev), topk, route_scale=2.5,
                       image_mask=torch.from_numpy(mask).to(dev), gate_b_vl=to_dev(gate_b_vl, dev))
    torch.cuda.synchronize()
    zn = z.cpu().numpy().copy()
    _check_logits(zn, xt.float().cpu().numpy(), gate_w)
    for r in range(rows):
        ridx, rw = coop.route(zn[r:r + 1], topk, "sqrt_softplus", gate_b_vl if mask[r] else gate_b, 2.5)
        assert np.array_equal(idx[r].cpu().numpy(), ridx[0]), r
        assert np.array_equal(w[r].cpu().numpy(), rw[0]), r
    # the standalone gate GEMV and the fused one are the same kernel: bit-identical logits
    ws = ops.MoeWorkspace(dev, rows_max=rows, hidden=H, inter=2048, topk=topk, n_local=E, has_shared=False)
    dummy = DeviceExperts([synth.expert(rng, H, 2048, 2, 1 / np.sqrt(H))], dev)
    sel = torch.empty(rows, topk, dtype=torch.int64, device=dev)
    wt = torch.empty(rows, topk, dtype=torch.float32, device=dev)
    out = torch.empty(rows, H, dtype=torch.float32, device=dev)
    ops.moe_forward(ws, xt, dummy.table[:, :1].expand(9, E).contiguous(), out, limit=10.0, bits=2,
                    gate_w=to_dev(gate_w, dev), sel=sel, weights=wt)
    torch.cuda.synchronize()
    assert np.array_equal(ws.logits(rows, E).cpu().numpy().view(np.uint32), zn.view(np.uint32))


def test_router_logits_round_bf16_x_to_fp16(dev):
    """Block.experts routes on ``x.to(float16)`` (model.py:455, then x.float() @ gate_w at
    :404-409): bf16 activations are rounded to fp16 first. Row 1 lies in the fp16 subnormal range
    (about 4 significant bits there), so the rounding moves its logits far outside the fp32
    accumulation bound; row 2 holds 70000, inf in fp16, so its logits are infinite."""
    ops = _ops()
    H, E = 1024, 64
    rng = np.random.default_rng(12)
    x = synth.activations_bf16(rng, 3, H)
    x[1] = coop.round_bf16(x[1] * 2.0e-6)
    x[2, 100] = 70000.0
    gate_w = _gate(rng, E, H)
    z = ops.router_logits(to_dev(x, dev).to(torch.bfloat16), to_dev(gate_w, dev)).cpu().numpy()
    xh = x.astype(np.float16).astype(np.float32)
    _check_logits(z[:2], xh[:2], gate_w)
    with pytest.raises(AssertionError):                  # the unrounded values miss the bound
        _check_logits(z[1:2], x[1:2], gate_w)
    assert np.all(np.isinf(z[2])) and np.array_equal(np.sign(z[2]), np.sign(gate_w[:, 100]))
