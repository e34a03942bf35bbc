"""evamx_moe_forward_static (the entry point that allocates nothing: the forward on the
library's fixed device scratch) against evamx_moe_forward with a caller's workspace, through
the C ABI: two calls in a row on the same GPU, the second with fewer rows, each bit-identical to
the workspace path on the same inputs (same shape, so the same layout and work split), and the
first also against the oracle. Plus the refusals: a shape too large for the scratch, and a
workspace argument."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import coop, synth
from tests.gpu_helpers import DeviceExperts, rel_err_rows, to_dev

pytestmark = pytest.mark.gpu
H, I, E, TOPK, ROWS_MAX = 512, 256, 24, 4, 16


@pytest.fixture(scope="module")
def case(dev):
    rng = np.random.default_rng(808)
    experts = [synth.expert(rng, H, I, 4, 1 / np.sqrt(H)) for _ in range(E)]
    shared = synth.expert(rng, H, I, 4, 1 / np.sqrt(H))
    return experts, shared, DeviceExperts(experts, dev), DeviceExperts([shared], dev)


def _run(ops, dev, case, x, logits, static, rows_max=ROWS_MAX):
    experts, shared, de, ds = case
    rows = x.shape[0]
    sel = torch.full((rows, TOPK), -1, dtype=torch.int64, device=dev)
    w = torch.full((rows, TOPK), -1.0, dtype=torch.float32, device=dev)
    out = torch.full((rows, H), float("nan"), dtype=torch.float32, device=dev)
    kw = dict(limit=0.75, bits=4, logits=to_dev(logits, dev), sel=sel, weights=w, shared_ptrs=ds.ptrs(0),
              shared_bits=4)
    xt = to_dev(x, dev).to(torch.bfloat16)
    if static:
        ops.moe_forward_static(ops.MoeShape(rows_max, H, I, TOPK, E, 1, 0, 0, 0), xt, de.table, out, **kw)
    else:
        ws = ops.MoeWorkspace(dev, rows_max=rows_max, hidden=H, inter=I, topk=TOPK, n_local=E, has_shared=True)
        ws.buffer.fill_(0x7f)
        ws.clear_flags()
        ops.moe_forward(ws, xt, de.table, out, **kw)
    torch.cuda.synchronize()
    return out.cpu().numpy(), sel.cpu().numpy(), w.cpu().numpy()


def test_static_forward_captured_in_a_graph(dev, case):
    """The entry point as the callers it is for use it: static forwards of 1, 2 and 16 rows (the
    one-row launch that routes inside, the two-row decode path, the 16-row MFMA tiles) captured
    into one hipGraph. First in this file, so that in a fresh process the per-device set-up
    (symbol lookup and the flag word's fill kernel) happens under capture. Three replays, with
    eager static calls of other sizes in between that overwrite the scratch, each equal bit for
    bit to the eager static calls and to the workspace path on the same inputs."""
    from eva_amd import ops
    experts, shared, de, ds = case
    rng = np.random.default_rng(811)
    shape = ops.MoeShape(ROWS_MAX, H, I, TOPK, E, 1, 0, 0, 0)
    calls = []
    for rows in (1, 2, 16):
        x = to_dev(synth.activations_bf16(rng, rows, H), dev).to(torch.bfloat16)
        z = to_dev(synth.logits_skewed(rng, rows, E, hot=1, warm=3), dev)
        bufs = dict(sel=torch.empty(rows, TOPK, dtype=torch.int64, device=dev),
                    weights=torch.empty(rows, TOPK, dtype=torch.float32, device=dev))
        out = torch.empty(rows, H, dtype=torch.float32, device=dev)
        calls.append((x, z, bufs, out))

    def run_all():
        for x, z, bufs, out in calls:
            ops.moe_forward_static(shape, x, de.table, out, limit=0.75, bits=4, logits=z, shared_ptrs=ds.ptrs(0),
                                   shared_bits=4, **bufs)

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run_all()
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    graph_out = [out.clone() for _, _, _, out in calls]
    for _, _, _, out in calls:
        out.fill_(float("nan"))
    run_all()                                                     # eager static calls
    torch.cuda.synchronize()
    for (x, z, bufs, out), got in zip(calls, graph_out):
        assert torch.equal(out.view(torch.int32), got.view(torch.int32))
        ws = ops.MoeWorkspace(dev, rows_max=ROWS_MAX, hidden=H, inter=I, topk=TOPK, n_local=E, has_shared=True)
        want = torch.empty_like(out)
        ops.moe_forward(ws, x, de.table, want, limit=0.75, bits=4, logits=z, shared_ptrs=ds.ptrs(0), shared_bits=4,
                        sel=torch.empty_like(bufs["sel"]), weights=torch.empty_like(bufs["weights"]))
        torch.cuda.synchronize()
        assert torch.equal(want.view(torch.int32), got.view(torch.int32))
    other = synth.activations_bf16(rng, 5, H)
    for rows in (5, 3, 9):                                        # eager work on the scratch between replays
        _run(ops, dev, case, other[:min(rows, 5)], synth.logits_plain(rng, min(rows, 5), E), static=True)
        for _, _, _, out in calls:
            out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for (_, _, _, out), got in zip(calls, graph_out):
            assert torch.equal(out.view(torch.int32), got.view(torch.int32))


def test_static_scratch_matches_workspace_twice(dev, case):
    from eva_amd import ops
    experts, shared, _, _ = case
    rng = np.random.default_rng(809)
    for n, rows in enumerate((ROWS_MAX, 3)):                 # the second call is smaller
        x = synth.activations_bf16(rng, rows, H)
        logits = synth.logits_skewed(rng, rows, E, hot=1, warm=3)
        got = _run(ops, dev, case, x, logits, static=True)
        want = _run(ops, dev, case, x, logits, static=False)
        for g, w in zip(got, want):
            assert np.array_equal(g.view(np.uint32) if g.dtype == np.float32 else g,
                                  w.view(np.uint32) if w.dtype == np.float32 else w), (n, rows)
        ref, ridx, _, _ = coop.moe_layer(x, logits, experts, shared, TOPK, 0.75)
        assert np.array_equal(got[1], ridx)
        assert rel_err_rows(got[0], ref) < 1e-2


def test_static_scratch_past_16_rows(dev, case):
    """Past 16 rows the workspace path pipelines its two tile size classes on the thread's side
    stream, while the fixed-scratch entry point creates no stream and runs every stage on the
    caller's: both give the same bits, at 40 rows and then 20 (both calls on the MFMA path)."""
    from eva_amd import ops
    experts, shared, _, _ = case
    rng = np.random.default_rng(810)
    for n, rows in enumerate((40, 20)):
        x = synth.activations_bf16(rng, rows, H)
        logits = synth.logits_skewed(rng, rows, E, hot=1, warm=3)
        got = _run(ops, dev, case, x, logits, static=True, rows_max=40)
        want = _run(ops, dev, case, x, logits, static=False, rows_max=40)
        for g, w in zip(got, want):
            assert np.array_equal(g.view(np.uint32) if g.dtype == np.float32 else g,
                                  w.view(np.uint32) if w.dtype == np.float32 else w), (n, rows)
        ref, ridx, _, _ = coop.moe_layer(x, logits, experts, shared, TOPK, 0.75)
        assert np.array_equal(got[1], ridx)
        assert rel_err_rows(got[0], ref) < 1e-2


def test_static_refusals(dev, case):
    from eva_amd import _lib, ops
    L = _lib.lib()
    a = _lib.MoeArgs()
    a.shape = _lib.MoeShape(4096, 7168, 2048, 8, 256, 1, 0, 0, 0)     # a prefill-size workspace: too big
    a.rows = 1
    assert L.evamx_moe_forward_static(ctypes.byref(a), None) == _lib.EVAMX_ENOSPACE
    assert b"fixed scratch" in L.evamx_last_error()
    a.shape = _lib.MoeShape(1, H, I, TOPK, E, 0, 0, 0, 0)
    a.workspace = 1 << 20
    a.workspace_bytes = 1 << 20
    assert L.evamx_moe_forward_static(ctypes.byref(a), None) == _lib.EVAMX_EINVAL


def _strict_static(dev, de, ds, inter, seed):
    from eva_amd import ops
    rng = np.random.default_rng(seed)
    kw = dict(limit=0.75, bits=4, shared_ptrs=ds.ptrs(0), shared_bits=4)

    def static(x, z, strict_rows):
        rows = x.shape[0]
        out = torch.empty(rows, H, dtype=torch.float32, device=dev)
        ops.moe_forward_static(ops.MoeShape(ROWS_MAX, H, inter, TOPK, E, 1, 0, 0, strict_rows), x, de.table, out,
                               logits=z, sel=torch.empty(rows, TOPK, dtype=torch.int64, device=dev),
                               weights=torch.empty(rows, TOPK, dtype=torch.float32, device=dev), **kw)
        torch.cuda.synchronize()
        return out

    for rows in (ROWS_MAX, 8):
        x = to_dev(synth.activations_bf16(rng, rows, H), dev).to(torch.bfloat16)
        z = to_dev(synth.logits_skewed(rng, rows, E, hot=1, warm=3), dev)
        got = static(x, z, ROWS_MAX)
        ws = ops.MoeWorkspace(dev, rows_max=ROWS_MAX, hidden=H, inter=inter, topk=TOPK, n_local=E, has_shared=True,
                              strict_rows=ROWS_MAX)
        want = torch.empty_like(got)
        ops.moe_forward(ws, x, de.table, want, logits=z, sel=torch.empty(rows, TOPK, dtype=torch.int64, device=dev),
                        weights=torch.empty(rows, TOPK, dtype=torch.float32, device=dev), **kw)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32), want.view(torch.int32)), rows
        for r in range(rows):
            alone = static(x[r:r + 1], z[r:r + 1], ROWS_MAX)
            assert torch.equal(alone.view(torch.int32), got[r:r + 1].view(torch.int32)), (rows, r)


def test_static_strict_rows(dev, case):
    """Strict mode on the fixed scratch: a 16-row static call with strict_rows 16 gives the bits of
    the workspace path in strict mode, and each of its rows the bits of a one-row static call (the
    strict property), then an 8-row call the bits of its own rows alone."""
    experts, shared, de, ds = case
    _strict_static(dev, de, ds, I, 812)


def test_static_strict_rows_paired_chunks(dev):
    """The same at I = 512 (four column groups), where the 16-row call pairs each expert's 8-row
    chunks (the hot expert's 16 rows and the shared expert's) in gate/up and down."""
    rng = np.random.default_rng(813)
    experts = [synth.expert(rng, H, 512, 4, 1 / np.sqrt(H)) for _ in range(E)]
    shared = synth.expert(rng, H, 512, 4, 1 / np.sqrt(H))
    _strict_static(dev, DeviceExperts(experts, dev), DeviceExperts([shared], dev), 512, 814)


@pytest.mark.parametrize("seed", range(6))
def test_static_random_configurations(dev, seed):
    """Seeded random shapes (widths of 2-8 chunks of 128, any expert count and top-k, mixed gate/up
    and down rates, a shared expert or none, strict or automatic geometry): two calls in a row on
    the fixed scratch, the second with fewer rows, each bit-identical to the workspace path."""
    from eva_amd import ops
    rng = np.random.default_rng(820 + seed)
    h, i = 128 * int(rng.integers(2, 9)), 128 * int(rng.integers(2, 9))
    e = int(rng.integers(4, 33))
    k = int(rng.integers(1, min(8, e) + 1))
    rows_max = int(rng.choice([2, 5, 16, 24, 40]))
    strict = rows_max if rows_max * k <= 256 and rng.random() < 0.5 else 0
    has_shared = bool(rng.random() < 0.7)
    rates = (1.5, 2, 2.5, 3, 3.5, 4, 5)
    experts = [synth.expert(rng, h, i, float(rng.choice(rates)), 1 / np.sqrt(h), K_down=float(rng.choice(rates)))
               for _ in range(e)]
    de = DeviceExperts(experts, dev)
    kw = dict(limit=10.0, k2_per_expert=de.k2, k2_down_per_expert=de.k2_down)
    if has_shared:
        ds = DeviceExperts([synth.expert(rng, h, i, 3.0, 1 / np.sqrt(h))], dev)
        kw.update(shared_ptrs=ds.ptrs(0), shared_bits=3.0)
    shape = ops.MoeShape(rows_max, h, i, k, e, int(has_shared), 0, 0, strict)
    print("case", seed, dict(h=h, i=i, e=e, k=k, rows_max=rows_max, strict=strict, shared=has_shared), flush=True)
    for n, rows in enumerate((rows_max, max(1, rows_max // 3))):
        x = to_dev(synth.activations_bf16(rng, rows, h), dev).to(torch.bfloat16)
        z = to_dev(synth.logits_zipf(rng, rows, e), dev)
        res = []
        for static in (True, False):
            sel = torch.full((rows, k), -1, dtype=torch.int64, device=dev)
            w = torch.full((rows, k), -1.0, dtype=torch.float32, device=dev)
            out = torch.full((rows, h), float("nan"), dtype=torch.float32, device=dev)
            if static:
                ops.moe_forward_static(shape, x, de.table, out, logits=z, sel=sel, weights=w, **kw)
            else:
                ws = ops.MoeWorkspace(dev, rows_max=rows_max, hidden=h, inter=i, topk=k, n_local=e,
                                      has_shared=has_shared, strict_rows=strict)
                ws.buffer.fill_(0x7f)
                ws.clear_flags()
                ops.moe_forward(ws, x, de.table, out, logits=z, sel=sel, weights=w, **kw)
            torch.cuda.synchronize()
            res.append((out.cpu().numpy(), sel.cpu().numpy(), w.cpu().numpy()))
        for g, want in zip(*res):
            assert np.array_equal(g.view(np.uint32) if g.dtype == np.float32 else g,
                                  want.view(np.uint32) if want.dtype == np.float32 else want), (n, rows)
        assert np.isfinite(res[0][0]).all()
