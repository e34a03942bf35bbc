"""A DS41PK01 pack loaded into HBM and run through the all-resident expert store, against the
CPU oracle on the same experts: given routes (ExpertCache.moe, cache.py:2276) and a routed
step with the shared expert. Mixed rates, including half rates, in one layer."""
import numpy as np
import pytest
import torch

from eva_amd import pack
from oracle import coop, synth
from tests.gpu_helpers import DeviceExperts, rel_err_rows, to_dev

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _pack(tmp_path, rng, H, I, rates):
    layers, oracle_layers = [], []
    for row in rates:
        exps, ors = [], []
        for K in row:
            ew = synth.expert(rng, H, I, K, 1 / np.sqrt(H))
            part = lambda p: (ew.parts[p][1], ew.parts[p][2], ew.parts[p][0])
            exps.append({"w1": part("g"), "w2": part("d"), "w3": part("u")})
            ors.append(ew)
        layers.append(exps)
        oracle_layers.append(ors)
    path = str(tmp_path / "experts.bin")
    pack.write_pack(path, layers)
    return path, oracle_layers


def test_resident_store_matches_oracle(dev, tmp_path):
    from eva_amd.cache import ResidentExperts
    rng = np.random.default_rng(31)
    H, I, topk, T, limit = 512, 256, 4, 5, 10.0
    rates = [[2, 2.5, 3, 4, 5, 3.5, 4, 1.5], [4] * 8]
    path, oracle_layers = _pack(tmp_path, rng, H, I, rates)
    store = ResidentExperts(path, dev, topk=topk, max_rows=8)
    assert tuple(store.packed.shape) == (2, 9, 8) and (store.hidden, store.inter) == (H, I)
    for l, res in store._layers.items():
        lo, hi = res.storage.data_ptr(), res.storage.data_ptr() + res.storage.numel()
        assert bool(((store.packed[l] >= lo) & (store.packed[l] < hi)).all())
        assert res.k2_host == tuple(int(2 * k) for k in rates[l])

    # given routes, mixed-rate layer
    x = synth.activations_bf16(rng, T, H).astype(np.float16)
    logits = synth.logits_plain(rng, T, 8)
    ridx, rw = coop.route(logits, topk)
    y = store.moe(0, to_dev(x, dev), to_dev(ridx, dev), to_dev(rw, dev), None, limit, I)
    torch.cuda.synchronize()
    ref = coop.moe_routed(x, ridx, rw.astype(np.float16), oracle_layers[0], limit)
    assert rel_err_rows(y.cpu().numpy(), ref) < TOL
    with pytest.raises(ValueError):
        store.moe(0, to_dev(x, dev), to_dev(ridx, dev), to_dev(rw, dev), 4, limit, I)     # mixed rates, k=4
    y1 = store.moe(1, to_dev(x, dev), to_dev(ridx, dev), to_dev(rw, dev), 4, limit, I)   # uniform 4 bpw
    ref1 = coop.moe_routed(x, ridx, rw.astype(np.float16), oracle_layers[1], limit)
    assert rel_err_rows(y1.cpu().numpy(), ref1) < TOL

    # routed step from logits with the shared expert, into a bf16 residual
    shared = synth.expert(rng, H, I, 4, 1 / np.sqrt(H))
    ds = DeviceExperts([shared], dev)
    xb = synth.activations_bf16(rng, T, H)
    out, sel, w = store.moe_step(0, to_dev(xb, dev).to(torch.bfloat16), to_dev(logits, dev), limit=limit,
                                 shared=ds.ptrs(0), shared_bits=4.0)
    torch.cuda.synchronize()
    ref2, idx2, _, _ = coop.moe_layer(xb, logits, oracle_layers[0], shared, topk, limit)
    assert np.array_equal(sel.cpu().numpy(), idx2)
    assert rel_err_rows(out.cpu().numpy(), ref2) < TOL
    assert store.flags(topk, True) == 0

    # the same step routed from the router weight: the routes are the oracle's routes of the
    # logits the kernel computed, into a residual stream updated in place
    gate_w = (rng.standard_normal((8, H)) / np.sqrt(H)).astype(np.float32)
    h0 = synth.activations_bf16(rng, T, H)
    h = to_dev(h0, dev).to(torch.bfloat16)
    _, sel3, _ = store.moe_step(0, h.clone(), gate_w=to_dev(gate_w, dev), limit=limit, shared=ds.ptrs(0),
                                shared_bits=4.0, residual=h, score_fn="sqrt_softplus")
    torch.cuda.synchronize()
    z = store._ws[(topk, True)].logits(T, 8).cpu().numpy().copy()
    ref3, idx3, _, _ = coop.moe_layer(h0, z, oracle_layers[0], shared, topk, limit,
                                      score_fn="sqrt_softplus")
    assert np.array_equal(sel3.cpu().numpy(), idx3)
    want = coop.residual_add(h0, ref3)
    got = h.float().cpu().numpy()
    # one bf16 rounding of the sum, plus the layer tolerance on the layer's contribution
    bound = np.maximum(np.abs(want), np.abs(got)) * 2.0 ** -8 + TOL * np.abs(ref3).max()
    assert np.all(np.abs(got - want) <= bound)
    with pytest.raises(ValueError):
        store.moe_step(0, h, to_dev(logits, dev), gate_w=to_dev(gate_w, dev))
