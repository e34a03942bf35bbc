"""The drop-in runners (eva_amd.coop, eva_amd.linear) on the GPU: results against the oracle,
and the reference's ownership rules (runtime/ds41/moe_coop3072.py:261-402)."""
import threading

import numpy as np
import pytest
import torch

from oracle import coop, synth
from tests.gpu_helpers import DeviceExperts, rel_err_rows, to_dev

pytestmark = pytest.mark.gpu
TOL = 1e-2
H, I, E = 256, 128, 12


@pytest.fixture(scope="module")
def case(dev):
    rng = np.random.default_rng(61)
    ex = [synth.expert(rng, H, I, 3, 1 / np.sqrt(H)) for _ in range(E)]
    return ex, DeviceExperts(ex, dev)


def _routes(rng, rows, topk):
    sel = np.stack([rng.choice(E, size=topk, replace=False) for _ in range(rows)]).astype(np.int64)
    w = rng.uniform(0.05, 1.0, size=(rows, topk)).astype(np.float32)
    return sel, w


def test_coop_runner_borrowed_output(dev, case):
    from eva_amd.coop import CoopRunner
    ex, de = case
    rng = np.random.default_rng(62)
    r = CoopRunner(dev, topk=4, hidden=H, inter=I, rows=2)
    x = rng.standard_normal((2, H)).astype(np.float16)
    sel, w = _routes(rng, 2, 4)
    rows = [de.table[i] for i in range(9)]                     # nine row views of one table
    y1 = r.run(to_dev(x, dev), to_dev(sel, dev).to(torch.int32), to_dev(w, dev), rows, 3, 10.0)
    torch.cuda.synchronize()
    ref = coop.moe_routed(x, sel, w.astype(np.float16), ex, 10.0)
    assert rel_err_rows(y1.cpu().numpy(), ref) < TOL
    y2 = r.run(to_dev(x, dev), to_dev(sel, dev), to_dev(w, dev), de.table, 3, 10.0)
    assert y2 is y1                                            # borrowed, overwritten by the next call


def test_capacity_runner_run_prepare_table(dev, case):
    from eva_amd.coop import CoopRunner3072
    ex, de = case
    rng = np.random.default_rng(63)
    r = CoopRunner3072(dev, topk=6, hidden=H, inter=I, max_rows=20)
    for rows in (20, 7):
        x = rng.standard_normal((rows, H)).astype(np.float16)
        sel, w = _routes(rng, rows, 6)
        w[1, 2] = 0.0
        y = r.run(to_dev(x, dev), to_dev(sel, dev), to_dev(w, dev), de.table, 3, 10.0)
        rw16 = w.astype(np.float16)
        assert y.shape == (rows, H) and y.data_ptr() != r.out.data_ptr()   # owned copy (moe_coop3072.py:312)
        assert rel_err_rows(y.cpu().numpy(), coop.moe_routed(x, sel, rw16, ex, 10.0)) < TOL
        assert np.array_equal(r.run_table().cpu().numpy(), coop.reference_table(sel, rw16, capacity=20))
        t = r.prepare_routes(to_dev(sel, dev), to_dev(w, dev), E)
        assert np.array_equal(t.cpu().numpy(), coop.reference_table(sel, rw16, capacity=20))
        assert np.array_equal(r.run_table().cpu().numpy(), t.cpu().numpy())
    life = r.lifecycle()
    assert not life["failed"] and not life["closed"] and life["owner_thread_matches"]
    r.close()
    assert r.lifecycle()["closed"]
    with pytest.raises(RuntimeError):
        r.run(to_dev(x, dev), to_dev(sel, dev), to_dev(w, dev), de.table, 3, 10.0)


def test_capacity_runner_bounds_poison_and_owner(dev, case):
    from eva_amd.coop import CoopRunner512
    _, de = case
    rng = np.random.default_rng(64)
    r = CoopRunner512(dev, topk=2, hidden=H, inter=I)
    x = to_dev(rng.standard_normal((2, H)).astype(np.float16), dev)
    w = to_dev(np.full((2, 2), 0.5, np.float32), dev)
    good = to_dev(np.array([[0, 1], [2, 3]], np.int64), dev)
    errors = []
    th = threading.Thread(target=lambda: errors.append(pytest.raises(RuntimeError, r.run, x, good, w, de.table, 3, 1.0)))
    th.start()
    th.join()
    assert errors                                              # wrong thread refused
    with pytest.raises(ValueError):
        r.run(x, good, w, de.table, 6, 1.0)                    # unsupported rate: argument error
    y1 = r.run(x, good, w, de.table, 3, 1.0)
    assert y1.data_ptr() == r.out.data_ptr() and y1.shape == (2, H)   # borrowed rows (moe_coop512.py:248)
    bad = to_dev(np.array([[0, 1], [2, 99]], np.int64), dev)   # 99 is outside the 12-entry table
    with pytest.raises(RuntimeError, match="outside"):
        r.run(x, bad, w, de.table, 3, 1.0)
    assert r.lifecycle()["failed"]
    with pytest.raises(RuntimeError):
        r.run(x, good, w, de.table, 3, 1.0)                    # poisoned


def test_elinear_batch_invariant(dev):
    """Up to 16 rows (decode GEMV) each row alone gives the same bits as in a 16-row call; beyond
    (MFMA path) a row gives the same bits in calls of 17, 37 and 101 rows. Both within TOL of the
    oracle."""
    from eva_amd.linear import build_linear
    rng = np.random.default_rng(65)
    tr, suh, svh = synth.projection(rng, 512, 384, 4, svh_scale=1 / np.sqrt(512))
    lin = build_linear(torch.from_numpy(suh), torch.from_numpy(svh), torch.from_numpy(tr), None, device=dev)
    x = rng.standard_normal((101, 512)).astype(np.float16)
    ref = coop.exl3_linear(x, tr, suh, svh, 4)
    y16 = lin.forward(to_dev(x[:16], dev)).cpu().numpy()
    assert rel_err_rows(y16.astype(np.float32), ref[:16].astype(np.float32)) < TOL
    for i in (0, 5, 15):                                       # each row alone gives the same bits
        yi = lin.forward(to_dev(x[i:i + 1], dev)).cpu().numpy()
        assert np.array_equal(yi[0].view(np.uint16), y16[i].view(np.uint16))
    y101 = lin.forward(to_dev(x, dev)).cpu().numpy()
    assert rel_err_rows(y101.astype(np.float32), ref.astype(np.float32)) < TOL
    y37 = lin.forward(to_dev(x[20:57], dev)).cpu().numpy()
    y17 = lin.forward(to_dev(x[84:], dev)).cpu().numpy()
    assert np.array_equal(y37.view(np.uint16), y101[20:57].view(np.uint16))
    assert np.array_equal(y17.view(np.uint16), y101[84:].view(np.uint16))
