"""The HIP kernels against the committed golden vectors (no oracle at run time).

Bars: states / decoded weights, Hadamard, router and run table bit-exact; the layer within a
max row-relative error of 1e-2."""
import numpy as np
import pytest
import torch

from tests.golden.make_golden import LAYER, RATES, layer_experts, load, rate_tag
from tests.gpu_helpers import DeviceExperts, rel_err_rows, to_dev

pytestmark = pytest.mark.gpu
TOL = 1e-2


@pytest.fixture(scope="module")
def g():
    return load()


@pytest.mark.parametrize("K", RATES)
def test_golden_dequant_gpu(dev, g, K):
    from eva_amd import ops
    t = rate_tag(K)
    w = ops.exl3_dequant(to_dev(g[f"dq_K{t}_trellis"], dev), K).cpu().numpy()
    assert np.array_equal(w.view(np.uint16), g[f"dq_K{t}_W"].view(np.uint16))


def test_golden_router_and_runs_gpu(dev, g):
    from eva_amd import ops
    for fn in ("sigmoid", "sqrt_softplus"):
        bias = to_dev(g["route_bias"], dev) if fn == "sqrt_softplus" else None
        idx, w, rw = ops.route_topk(to_dev(g["route_logits"], dev), 4, fn, bias, 2.5)
        assert np.array_equal(idx.cpu().numpy(), g[f"route_{fn}_idx"])
        assert np.array_equal(w.cpu().numpy(), g[f"route_{fn}_w"])
    runs = ops.prepare_routes(to_dev(g["runs_sel"], dev), to_dev(g["runs_rw"], dev), 12, 10)
    assert np.array_equal(runs.cpu().numpy(), g["runs_table"])


def test_golden_layer_gpu(dev, g):
    from eva_amd import ops
    experts, shared = layer_experts(g)
    H, I, E, k, T = LAYER["H"], LAYER["I"], LAYER["E"], LAYER["topk"], LAYER["T"]
    de, ds = DeviceExperts(experts, dev), DeviceExperts([shared], dev)
    ws = ops.MoeWorkspace(dev, rows_max=T, hidden=H, inter=I, topk=k, n_local=E, has_shared=True)
    sel = torch.empty(T, k, dtype=torch.int64, device=dev)
    w = torch.empty(T, k, dtype=torch.float32, device=dev)
    rw = torch.empty(T, k, dtype=torch.float16, device=dev)
    out = torch.empty(T, H, dtype=torch.float32, device=dev)
    ops.moe_forward(ws, to_dev(g["layer_x"], dev).to(torch.bfloat16), de.table, out, limit=LAYER["limit"],
                    k2_per_expert=de.k2, logits=to_dev(g["layer_logits"], dev), sel=sel, weights=w, rw=rw,
                    shared_ptrs=ds.ptrs(0), shared_bits=float(shared.K))
    torch.cuda.synchronize()
    assert np.array_equal(sel.cpu().numpy(), g["layer_idx"])
    assert np.array_equal(rw.cpu().numpy().view(np.uint16), g["layer_rw"].view(np.uint16))
    assert rel_err_rows(out.cpu().numpy(), g["layer_y"]) < TOL
