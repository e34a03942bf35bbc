"""Edge cases of the MoE forward on the GPU, against the CPU oracle: empty rows (no active slot:
shared term only, or zeros; exl3_moe_coop_kernel.cuh:573-610), expert ranges (EP filter,
exl3_moe_coop_kernel.cuh:208-223), the many-row grouping path, strided rows, workspace reuse
with a smaller call, and hipGraph replays (checked on every replay)."""
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
def test_empty_rows(dev, shared):
    from eva_amd import ops
    H, I, E, k, T = 256, 128, 6, 2, 4
    rng = np.random.default_rng(31)
    ex = _experts(rng, H, I, E, 3)
    sh = synth.expert(rng, H, I, 3, 1 / np.sqrt(H))
    x = rng.standard_normal((T, H)).astype(np.float16)
    sel = np.array([[0, 1], [2, 3], [4, 5], [1, 2]], dtype=np.int64)
    rw = np.array([[0.5, 0.5], [0, 0], [0.25, 0.75], [0, 0]], dtype=np.float16)   # rows 1, 3 empty
    ref = coop.moe_routed(x, sel, rw, ex, 10.0)
    if shared:
        ref = ref + coop.shared_expert(x, sh, 10.0)
    de, ds = DeviceExperts(ex, dev), DeviceExperts([sh], dev)
    ws = ops.MoeWorkspace(dev, rows_max=T, hidden=H, inter=I, topk=k, n_local=E, has_shared=shared)
    out = torch.full((T, H), float("nan"), dtype=torch.float32, device=dev)
    ops.moe_forward(ws, to_dev(x, dev), de.table, out, limit=10.0, bits=3, sel=to_dev(sel, dev), rw=to_dev(rw, dev),
                    shared_ptrs=ds.ptrs(0) if shared else None, shared_bits=3 if shared else None)
    torch.cuda.synchronize()
    y = out.cpu().numpy()
    assert np.all(np.isfinite(y))
    if not shared:
        assert np.all(y[1] == 0) and np.all(y[3] == 0)
    assert rel_err_rows(y, ref) < TOL


def test_expert_range(dev):
    from eva_amd import ops
    H, I, k, T = 256, 128, 4, 6
    lo, hi = 4, 12
    rng = np.random.default_rng(32)
    ex = _experts(rng, H, I, hi - lo, 2)
    x = rng.standard_normal((T, H)).astype(np.float16)
    sel = np.stack([rng.choice(16, size=k, replace=False) for _ in range(T)]).astype(np.int64)
    rw = rng.uniform(0.1, 1, size=(T, k)).astype(np.float16)
    ref = coop.moe_routed(x, sel, rw, ex, 0.0, min_expert=lo, max_expert=hi)
    de = DeviceExperts(ex, dev)
    ws = ops.MoeWorkspace(dev, rows_max=T, hidden=H, inter=I, topk=k, n_local=hi - lo, has_shared=False)
    out = torch.empty(T, H, dtype=torch.float32, device=dev)
    ops.moe_forward(ws, to_dev(x, dev), de.table, out, limit=0.0, bits=2, sel=to_dev(sel, dev), rw=to_dev(rw, dev),
                    min_expert=lo, max_expert=hi)
    torch.cuda.synchronize()
    assert int(ws.flags().cpu()[0]) == 0                          # out-of-range picks are not errors here
    assert rel_err_rows(out.cpu().numpy(), ref) < TOL
    ok, _ = coop.slot_active(sel, rw, lo, hi)
    assert np.array_equal(ws.runs().cpu().numpy(), coop.reference_table(np.where(ok, sel - lo, 0), np.where(ok, rw, 0),
                                                                        capacity=T))


def test_many_rows_strided(dev):
    """40 rows take the single-workgroup grouping path; x and out are row-strided views."""
    from eva_amd import ops
    H, I, E, k, T = 256, 128, 12, 4, 40
    rng = np.random.default_rng(33)
    ex = _experts(rng, H, I, E, 4)
    sh = synth.expert(rng, H, I, 4, 1 / np.sqrt(H))
    x = synth.activations_bf16(rng, T, H)
    logits = synth.logits_skewed(rng, T, E, hot=1, warm=3)
    ref, ridx, _, rrw = coop.moe_layer(x, logits, ex, sh, k, 10.0)
    de, ds = DeviceExperts(ex, dev), DeviceExperts([sh], dev)
    ws = ops.MoeWorkspace(dev, rows_max=64, hidden=H, inter=I, topk=k, n_local=E, has_shared=True)
    xw = torch.zeros(T, H + 128, dtype=torch.bfloat16, device=dev)
    xw[:, :H] = to_dev(x, dev).to(torch.bfloat16)
    ow = torch.full((T, H + 64), 7.0, dtype=torch.float32, device=dev)
    sel = torch.empty(T, k, dtype=torch.int64, device=dev)
    w = torch.empty(T, k, dtype=torch.float32, device=dev)
    ops.moe_forward(ws, xw[:, :H], de.table, ow[:, :H], limit=10.0, bits=4, logits=to_dev(logits, dev), sel=sel,
                    weights=w, shared_ptrs=ds.ptrs(0), shared_bits=4)
    torch.cuda.synchronize()
    assert np.array_equal(sel.cpu().numpy(), ridx)
    assert np.array_equal(ws.runs().cpu().numpy(), coop.reference_table(ridx, rrw, capacity=64))
    o = ow.cpu().numpy()
    assert np.all(o[:, H:] == 7.0)                                # nothing written past the row
    assert rel_err_rows(o[:, :H], ref) < TOL


def test_workspace_reuse_smaller_call(dev):
    from eva_amd import ops
    H, I, E, k = 256, 256, 8, 2
    rng = np.random.default_rng(34)
    ex = _experts(rng, H, I, E, 5)
    de = DeviceExperts(ex, dev)
    ws = ops.MoeWorkspace(dev, rows_max=16, hidden=H, inter=I, topk=k, n_local=E, has_shared=False)
    for T in (16, 3):
        x = rng.standard_normal((T, H)).astype(np.float16)
        sel = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int64)
        rw = rng.uniform(0.1, 1, size=(T, k)).astype(np.float16)
        out = torch.empty(T, H, dtype=torch.float32, device=dev)
        ops.moe_forward(ws, to_dev(x, dev), de.table, out, limit=10.0, bits=5, sel=to_dev(sel, dev), rw=to_dev(rw, dev))
        torch.cuda.synchronize()
        assert rel_err_rows(out.cpu().numpy(), coop.moe_routed(x, sel, rw, ex, 10.0)) < TOL
        assert np.array_equal(ws.runs().cpu().numpy(), coop.reference_table(sel, rw, capacity=16))   # no stale entries


def test_eager_call_during_another_capture(dev):
    """A 40-token forward captured on one stream joins the thread's side stream into that
    capture; an eager 40-token call the same thread makes on another stream before the capture
    ends must not fork onto it (it runs on its own stream), and both the eager result and the
    graph's replay equal a plain eager call."""
    from eva_amd import ops
    H, I, E, k, T = 256, 128, 16, 4, 40
    rng = np.random.default_rng(36)
    ex = _experts(rng, H, I, E, 4)
    sh = synth.expert(rng, H, I, 4, 1 / np.sqrt(H))
    de, ds = DeviceExperts(ex, dev), DeviceExperts([sh], dev)
    x = to_dev(synth.activations_bf16(rng, T, H), dev).to(torch.bfloat16)
    z = to_dev(synth.logits_plain(rng, T, E), dev)

    def make():
        ws = ops.MoeWorkspace(dev, rows_max=T, hidden=H, inter=I, topk=k, n_local=E, has_shared=True)
        sel = torch.empty(T, k, dtype=torch.int64, device=dev)
        w = torch.empty(T, k, dtype=torch.float32, device=dev)
        out = torch.empty(T, H, dtype=torch.float32, device=dev)
        return lambda: ops.moe_forward(ws, x, de.table, out, limit=10.0, bits=4, logits=z, sel=sel, weights=w,
                                       shared_ptrs=ds.ptrs(0), shared_bits=4), out

    f_ref, out_ref = make()
    f_ref()                                             # eager: creates the side stream
    torch.cuda.synchronize()
    f_cap, out_cap = make()
    f_eager, out_eager = make()
    other = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        f_cap()
        with torch.cuda.stream(other):
            f_eager()                                   # eager, while the side stream is in the capture
    torch.cuda.synchronize()
    assert torch.equal(out_eager, out_ref)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out_cap, out_ref)


@pytest.mark.parametrize("T", [2, 40])
def test_graph_replays(dev, T):
    """Captured forward (routing included), replayed with new inputs copied into the static
    buffers between replays; every replay equals the eager result for the same inputs. At 40
    tokens the MFMA stages run their two kernels concurrently (the side stream joins the
    capture)."""
    from eva_amd import ops
    H, I, E, k = 256, 128, 16, 4
    rng = np.random.default_rng(35)
    ex = _experts(rng, H, I, E, 4)
    sh = synth.expert(rng, H, I, 4, 1 / np.sqrt(H))
    de, ds = DeviceExperts(ex, dev), DeviceExperts([sh], dev)
    ws = ops.MoeWorkspace(dev, rows_max=T, hidden=H, inter=I, topk=k, n_local=E, has_shared=True)
    xs = torch.zeros(T, H, dtype=torch.bfloat16, device=dev)
    zs = torch.zeros(T, E, dtype=torch.float32, device=dev)
    sel = torch.empty(T, k, dtype=torch.int64, device=dev)
    w = torch.empty(T, k, dtype=torch.float32, device=dev)
    out = torch.empty(T, H, dtype=torch.float32, device=dev)

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
        x = synth.activations_bf16(rng, T, H)
        z = synth.logits_plain(rng, T, E)
        xs.copy_(to_dev(x, dev).to(torch.bfloat16))
        zs.copy_(to_dev(z, dev))
        graph.replay()
        torch.cuda.synchronize()
        y_graph = out.clone()
        idx_graph = sel.clone()
        fwd()                                                     # eager on the same inputs
        torch.cuda.synchronize()
        assert torch.equal(idx_graph, sel), rep
        assert torch.equal(y_graph, out), rep
        ref, ridx, _, _ = coop.moe_layer(x, z, ex, sh, k, 10.0)
        assert np.array_equal(idx_graph.cpu().numpy(), ridx)
        assert rel_err_rows(y_graph.cpu().numpy(), ref) < TOL


def test_decode_ceiling_benchmark(dev):
    """The register-only decode benchmark runs at every GEMV rate and reports a plausible rate
    (between 1e12 and 1e14 weights/s on one MI355X)."""
    from eva_amd import ops
    for bits in (1.5, 2.0, 2.5, 3.0, 3.5, 4.0, 5.0):
        wps = ops.decode_ceiling(bits, dev, iters=200)
        assert 1e12 < wps < 1e14, (bits, wps)


def test_read_floor_benchmark(dev):
    """The read-only benchmark runs in a small and in the one-row gate/up shape and reports a rate
    below HBM's 8 TB/s peak (the buffers are far larger than the caches at the full shape)."""
    from eva_amd import ops
    assert ops.read_floor(16, 8, 64, dev, reps=3) > 0
    bps = ops.read_floor(16, 64, 2016, dev, reps=5)
    assert 1e12 < bps < 8.5e12, bps
