"""The PyTorch-CPU restatement that bench.py times as the CPU baseline (oracle/torch_cpu.py)
computes the same layer as the parity oracle (oracle/coop.py), within the layer tolerance: it
keeps every operation and skips only the fp16 rounding points."""
import numpy as np
import pytest
import torch

from oracle import coop, synth, torch_cpu

TOL = 1e-2


def _parts(ew):
    return tuple(tuple(torch.from_numpy(np.ascontiguousarray(a)) for a in ew.parts[p]) for p in "gud")


@pytest.mark.parametrize("limit", [10.0, 0.75])
@pytest.mark.parametrize("K", [4, 2.5])
def test_torch_cpu_layer_matches_oracle(limit, K):
    H, I, E, topk, T = 512, 256, 12, 4, 3
    rng = np.random.default_rng(31 + int(2 * K))
    experts = [synth.expert(rng, H, I, K, 1 / np.sqrt(H)) for _ in range(E)]
    shared = synth.expert(rng, H, I, K, 1 / np.sqrt(H))
    x = synth.activations_bf16(rng, T, H)
    logits = synth.logits_skewed(rng, T, E, hot=1, warm=3)
    ref, idx, w, _ = coop.moe_layer(x, logits, experts, shared, topk, limit)
    dec = torch_cpu.Decoder(K)
    xt = torch.from_numpy(x.astype(np.float16).astype(np.float32))
    got = torch_cpu.moe_layer(xt, torch.from_numpy(idx), torch.from_numpy(w.astype(np.float16).astype(np.float32)),
                              {e: _parts(experts[e]) for e in range(E)}, _parts(shared), dec, limit)
    assert coop.rel_err_rows(got.numpy(), ref) < TOL


def test_torch_cpu_route_matches_oracle():
    rng = np.random.default_rng(33)
    z = rng.standard_normal((9, 256)).astype(np.float32)
    idx, w = torch_cpu.route_sigmoid(torch.from_numpy(z), 8)
    ridx, rw = coop.route(z, 8)
    assert np.array_equal(idx.numpy(), ridx)
    assert np.allclose(w.numpy(), rw, rtol=1e-6, atol=0)


def test_torch_cpu_linear_matches_oracle():
    rng = np.random.default_rng(34)
    tr, suh, svh = synth.projection(rng, 512, 384, 4, svh_scale=1 / np.sqrt(512))
    x = rng.standard_normal((2, 512)).astype(np.float16)
    ref = coop.exl3_linear(x, tr, suh, svh, 4).astype(np.float32)
    got = torch_cpu.linear_forward(torch.from_numpy(x.astype(np.float32)), *(torch.from_numpy(a) for a in (tr, suh, svh)),
                                   torch_cpu.Decoder(4))
    assert coop.rel_err_rows(got.numpy(), ref) < TOL
