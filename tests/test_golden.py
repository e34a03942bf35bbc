"""The CPU restatement still reproduces the committed golden vectors bit for bit
(tests/golden/make_golden.py wrote them from the pinned oracle)."""
import numpy as np
import pytest

from oracle import coop, exl3
from tests.golden.make_golden import LAYER, RATES, layer_experts, load, rate_tag


@pytest.fixture(scope="module")
def g():
    return load()


@pytest.mark.parametrize("K", RATES)
def test_golden_dequant(g, K):
    t = rate_tag(K)
    tr = g[f"dq_K{t}_trellis"]
    assert np.array_equal(exl3.trellis_states(tr, K), g[f"dq_K{t}_states"])
    assert np.array_equal(exl3.dequant(tr, K).view(np.uint16), g[f"dq_K{t}_W"].view(np.uint16))


def test_golden_hadamard_router_runs(g):
    assert np.array_equal(exl3.had128(g["had_v"]), g["had_y"])
    for fn in ("sigmoid", "sqrt_softplus"):
        idx, w = coop.route(g["route_logits"], 4, fn, g["route_bias"] if fn == "sqrt_softplus" else None, 2.5)
        assert np.array_equal(idx, g[f"route_{fn}_idx"])
        assert np.array_equal(w, g[f"route_{fn}_w"])
    assert np.array_equal(g["route_sigmoid_idx"][2], np.arange(4))
    assert np.array_equal(coop.reference_table(g["runs_sel"], g["runs_rw"], capacity=12), g["runs_table"])


def test_golden_layer(g):
    experts, shared = layer_experts(g)
    y, idx, _, rw = coop.moe_layer(g["layer_x"], g["layer_logits"], experts, shared, LAYER["topk"], LAYER["limit"])
    assert np.array_equal(idx, g["layer_idx"])
    assert np.array_equal(rw.view(np.uint16), g["layer_rw"].view(np.uint16))
    assert np.array_equal(y, g["layer_y"])
