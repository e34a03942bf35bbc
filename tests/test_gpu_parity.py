"""GPU parity of the HIP kernels against the CPU oracle, on identical seeded inputs.

Bars: decoded fp16 weights, router indices and run tables bit-exact; layer outputs within a
max row-relative error of 1e-2 (max_r max|y_r - ref_r| / max|ref_r|).
"""
import numpy as np
import pytest
import torch

from oracle import coop, exl3, synth
from tests.gpu_helpers import DeviceExperts, clamp_variants, rel_err_rows, to_dev

pytestmark = pytest.mark.gpu

TOL = 1e-2
CLIP = 0.75          # SwiGLU limit that clips ~12% of SiLU(G) and ~45% of U at these scales


def _assert_clamp_parity(y, variants):
    """y matches the reference clamp semantics and none of the wrong ones (the wrong ones sit
    far outside the tolerance at CLIP, so a kernel that skips or reorders a clamp fails)."""
    assert rel_err_rows(y, variants["ref"]) < TOL
    for name in ("routed_swapped", "shared_swapped", "unclamped"):
        assert rel_err_rows(variants[name], variants["ref"]) > 5 * TOL, name
        assert rel_err_rows(y, variants[name]) > 2 * TOL, name


def _ops():
    from eva_amd import ops
    return ops


@pytest.mark.parametrize("K", [2, 3, 4, 5, 1, 6, 8, 1.5, 2.5, 3.5])
def test_dequant_bit_exact(dev, K):
    ops = _ops()
    rng = np.random.default_rng(int(K * 10))
    n_in, n_out = 64, 256
    tr = rng.integers(-32768, 32768, size=(n_in // 16, n_out // 16, exl3.tile_u16(K)), dtype=np.int16)
    w = ops.exl3_dequant(to_dev(tr, dev), K).cpu().numpy()
    ref = exl3.dequant(tr, K)
    assert np.array_equal(w.view(np.uint16), ref.view(np.uint16))


def test_dequant_dsv3_projection_bit_exact(dev):
    ops = _ops()
    rng = np.random.default_rng(7)
    tr = rng.integers(-32768, 32768, size=(7168 // 16, 2048 // 16, 64), dtype=np.int16)
    w = ops.exl3_dequant(to_dev(tr, dev), 4).cpu().numpy()
    ref = coop.dequant_fast(tr, 4)
    assert np.array_equal(w.view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("score", ["sigmoid", "sqrt_softplus"])
@pytest.mark.parametrize("bias", [False, True])
def test_route_topk_bit_exact(dev, score, bias):
    ops = _ops()
    rng = np.random.default_rng(3)
    z = rng.standard_normal((37, 256)).astype(np.float32)
    z[5] = 0.25                                       # all-equal row -> indices 0..k-1
    z[6, 10:20] = 1.5                                 # ties inside the top-k
    b = rng.standard_normal(256).astype(np.float32) * 0.1 if bias else None
    idx, w, rw = ops.route_topk(to_dev(z, dev), 8, score, None if b is None else to_dev(b, dev), 2.5)
    ridx, rwt = coop.route(z, 8, score, b, 2.5)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert np.array_equal(w.cpu().numpy(), rwt)
    assert np.array_equal(rw.cpu().numpy(), rwt.astype(np.float16))
    if b is None:
        assert np.array_equal(ridx[5], np.arange(8))


@pytest.mark.parametrize("rows,topk,n_local,zero_frac", [(1, 8, 256, 0.0), (16, 8, 256, 0.1),
                                                          (512, 6, 384, 0.05), (64, 8, 12, 0.0)])
def test_prepare_routes_bit_exact(dev, rows, topk, n_local, zero_frac):
    ops = _ops()
    rng = np.random.default_rng(rows + topk)
    sel = np.stack([rng.choice(n_local, size=topk, replace=False) for _ in range(rows)]).astype(np.int64)
    rw = rng.uniform(0.05, 1.0, size=(rows, topk)).astype(np.float16)
    rw[rng.uniform(size=rw.shape) < zero_frac] = 0
    cap = rows + 3
    runs = ops.prepare_routes(to_dev(sel, dev), to_dev(rw, dev), cap, n_local).cpu().numpy()
    ref = coop.reference_table(sel, rw, capacity=cap)
    assert np.array_equal(runs, ref)


@pytest.mark.parametrize("K", [2, 3, 4, 5, 1.5, 2.5, 3.5])
@pytest.mark.parametrize("rows", [1, 3, 16])
def test_exl3_linear(dev, K, rows):
    ops = _ops()
    rng = np.random.default_rng(100 + rows)
    tr, suh, svh = synth.projection(rng, 512, 384, K, svh_scale=1 / np.sqrt(512))
    x = rng.standard_normal((rows, 512)).astype(np.float16)
    y = ops.exl3_linear(to_dev(x, dev), to_dev(tr, dev), to_dev(suh, dev), to_dev(svh, dev), K).cpu().numpy()
    ref = coop.exl3_linear(x, tr, suh, svh, K)
    assert rel_err_rows(y.astype(np.float32), ref.astype(np.float32)) < TOL


@pytest.mark.parametrize("shape", [(4096, 128), (7168, 256), (768, 128), (1280, 256)])
@pytest.mark.parametrize("rows", [1, 2, 5])
def test_exl3_linear_many_splits(dev, shape, rows):
    """Few output columns: the decode GEMV's k-split takes every 128-chunk of the input (32, 56, 6
    and 10 splits), so the epilogue sums its partials in several batches of 16, and with 6 and 10
    splits the last workgroup of a column group has waves past the last split (they only arrive)."""
    ops = _ops()
    n_in, n_out = shape
    rng = np.random.default_rng(n_in + rows)
    tr, suh, svh = synth.projection(rng, n_in, n_out, 4, svh_scale=1 / np.sqrt(n_in))
    x = rng.standard_normal((rows, n_in)).astype(np.float16)
    y = ops.exl3_linear(to_dev(x, dev), to_dev(tr, dev), to_dev(suh, dev), to_dev(svh, dev), 4).cpu().numpy()
    ref = coop.exl3_linear(x, tr, suh, svh, 4)
    assert rel_err_rows(y.astype(np.float32), ref.astype(np.float32)) < TOL


ARRIVE_REST = 0x3C6EF372        # high word of a column group's arrival counter at rest


@pytest.mark.parametrize("rows", [1, 2])
def test_exl3_linear_arrival_counters(dev, rows):
    """Up to 2 rows the linear is one launch whose column groups meet at arrival counters in the
    workspace. Whatever the workspace held before (all-ones bytes, zeros, random bytes, another
    shape's partials and counters), the first call gives the bits of a call on a settled
    workspace and leaves every counter at rest; so do graph replays of the call."""
    ops = _ops()
    n_in, n_out = 2048, 1024
    rng = np.random.default_rng(700 + rows)
    tr, suh, svh = synth.projection(rng, n_in, n_out, 4, svh_scale=1 / np.sqrt(n_in))
    x = rng.standard_normal((rows, n_in)).astype(np.float16)
    args = (to_dev(tr, dev), to_dev(suh, dev), to_dev(svh, dev), 4)
    xd = to_dev(x, dev)
    need = ops.lib().evamx_exl3_linear_workspace_bytes(rows, n_in, n_out)
    ncg = n_out // 128

    def at_rest(ws):                    # one counter per 128 bytes
        words = ws[: ncg * 128].view(torch.int64).cpu().numpy().astype(np.uint64)[::16]
        return bool(np.all(words == np.uint64(ARRIVE_REST << 32)))

    settled = torch.empty(need, dtype=torch.uint8, device=dev)
    ops.exl3_linear(xd, *args, workspace=settled)
    y0 = ops.exl3_linear(xd, *args, workspace=settled)
    torch.cuda.synchronize()
    assert at_rest(settled)
    ref = coop.exl3_linear(x, tr, suh, svh, 4)
    assert rel_err_rows(y0.cpu().numpy().astype(np.float32), ref.astype(np.float32)) < TOL

    g = torch.Generator(device=dev)
    g.manual_seed(rows)
    fills = {
        "ones": torch.full((need,), 0xFF, dtype=torch.uint8, device=dev),
        "zeros": torch.zeros(need, dtype=torch.uint8, device=dev),
        "random": torch.randint(0, 256, (need,), generator=g, dtype=torch.uint8, device=dev),
    }
    # another shape's call first: its partials and counters sit where this shape's counters are
    other = torch.empty(max(need, ops.lib().evamx_exl3_linear_workspace_bytes(1, 512, 7168)), dtype=torch.uint8,
                        device=dev)
    rng2 = np.random.default_rng(9)
    tr2, suh2, svh2 = synth.projection(rng2, 512, 7168, 4)
    ops.exl3_linear(to_dev(rng2.standard_normal((1, 512)).astype(np.float16), dev), to_dev(tr2, dev),
                    to_dev(suh2, dev), to_dev(svh2, dev), 4, workspace=other)
    fills["other shape"] = other
    for name, ws in fills.items():
        y = ops.exl3_linear(xd, *args, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(y, y0), name
        assert at_rest(ws), name

    ws = fills["random"]
    ws.copy_(torch.randint(0, 256, (ws.numel(),), generator=g, dtype=torch.uint8, device=dev))
    out = torch.empty_like(y0)
    s = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(s):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            ops.exl3_linear(xd, *args, out=out, workspace=ws)
    torch.cuda.synchronize()
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y0)
        assert at_rest(ws)


@pytest.mark.parametrize("K", [2, 3, 4, 5, 1.5, 2.5, 3.5])
@pytest.mark.parametrize("rows", [17, 64, 100])
def test_exl3_linear_mfma_path(dev, K, rows):
    """More than 16 rows: input rotation, then MFMA tiles whose waves sum their k-ranges in LDS
    and run the output epilogue (tiles of 17..64 rows and a ragged last tile)."""
    ops = _ops()
    rng = np.random.default_rng(200 + rows)
    tr, suh, svh = synth.projection(rng, 1024, 384, K, svh_scale=1 / np.sqrt(1024))
    x = rng.standard_normal((rows, 1024)).astype(np.float16)
    y = ops.exl3_linear(to_dev(x, dev), to_dev(tr, dev), to_dev(suh, dev), to_dev(svh, dev), K).cpu().numpy()
    ref = coop.exl3_linear(x, tr, suh, svh, K)
    assert rel_err_rows(y.astype(np.float32), ref.astype(np.float32)) < TOL


def _run_layer(ops, dev, x, logits, de, ds, H, I, E, topk, rows, limit, **kw):
    ws = ops.MoeWorkspace(dev, rows_max=rows, hidden=H, inter=I, topk=topk, n_local=E, has_shared=True)
    sel = torch.empty(rows, topk, dtype=torch.int64, device=dev)
    w = torch.empty(rows, topk, dtype=torch.float32, device=dev)
    out = torch.empty(rows, H, dtype=torch.float32, device=dev)
    ops.moe_forward(ws, to_dev(x, dev).to(torch.bfloat16), de.table, out, limit=limit, logits=to_dev(logits, dev),
                    sel=sel, weights=w, shared_ptrs=ds.ptrs(0), **kw)
    torch.cuda.synchronize()
    assert int(ws.flags().cpu()[0]) == 0
    return out.cpu().numpy(), sel.cpu().numpy()


@pytest.mark.parametrize("rows", [1, 2, 5, 40])
def test_moe_layer_down_rate_differs(dev, rows):
    """Gate/up and down at different rates (the reference launcher's K_gu and K_d,
    exl3_moe_coop.cuh:80-83): per-expert down-rate tables, a uniform down rate, and a shared
    expert whose down rate differs; through the decode GEMV (1-2 rows), the 16-row MFMA tiles
    (5) and the 64-row tiles (40)."""
    ops = _ops()
    H, I, E, topk, limit = 512, 256, 16, 4, 10.0
    rng = np.random.default_rng(300 + rows)
    pairs = [(4, 3), (3, 2), (2, 4), (2.5, 3.5), (4, 5), (1.5, 2), (3.5, 1.5), (5, 2.5)]
    experts = [synth.expert(rng, H, I, pairs[e % len(pairs)][0], svh_scale=1 / np.sqrt(H),
                            K_down=pairs[e % len(pairs)][1]) for e in range(E)]
    shared = synth.expert(rng, H, I, 4, svh_scale=1 / np.sqrt(H), K_down=3)
    x = synth.activations_bf16(rng, rows, H)
    logits = synth.logits_plain(rng, rows, E)
    ref, ridx, _, _ = coop.moe_layer(x, logits, experts, shared, topk, limit)
    de, ds = DeviceExperts(experts, dev), DeviceExperts([shared], dev)
    y, sel = _run_layer(ops, dev, x, logits, de, ds, H, I, E, topk, rows, limit, k2_per_expert=de.k2,
                        k2_down_per_expert=de.k2_down, shared_bits=4.0, shared_bits_down=3.0)
    assert np.array_equal(sel, ridx)
    assert rel_err_rows(y, ref) < TOL
    # uniform rates: gate/up 4, down 2.5
    experts_u = [synth.expert(rng, H, I, 4, svh_scale=1 / np.sqrt(H), K_down=2.5) for _ in range(E)]
    ref_u, _, _, _ = coop.moe_layer(x, logits, experts_u, shared, topk, limit)
    de_u = DeviceExperts(experts_u, dev)
    y_u, _ = _run_layer(ops, dev, x, logits, de_u, ds, H, I, E, topk, rows, limit, bits=4.0, bits_down=2.5,
                        shared_bits=4.0, shared_bits_down=3.0)
    assert rel_err_rows(y_u, ref_u) < TOL


@pytest.mark.parametrize("rows", [1, 2, 8, 40])
def test_moe_layer_gated_shared_expert(dev, rows):
    """Gated shared expert (exl3_moe_coop_kernel.cuh:881-903,942-948): the shared term scaled by
    sigmoid(x . w) per row, against the oracle; the gate visibly changes the output."""
    ops = _ops()
    H, I, E, topk, limit = 512, 256, 16, 4, 10.0
    rng = np.random.default_rng(400 + rows)
    experts, shared = _layer_case(rng, H, I, E, 4, 1 / np.sqrt(H))
    x = synth.activations_bf16(rng, rows, H)
    logits = synth.logits_plain(rng, rows, E)
    gw = (rng.standard_normal(H) * 0.08).astype(np.float16)
    ref, ridx, _, _ = coop.moe_layer(x, logits, experts, shared, topk, limit, shared_gate_w=gw)
    ungated, _, _, _ = coop.moe_layer(x, logits, experts, shared, topk, limit)
    assert rel_err_rows(ungated, ref) > 5 * TOL
    de, ds = DeviceExperts(experts, dev), DeviceExperts([shared], dev)
    y, sel = _run_layer(ops, dev, x, logits, de, ds, H, I, E, topk, rows, limit, bits=4.0, shared_bits=4.0,
                        shared_gate_w=to_dev(gw, dev))
    assert np.array_equal(sel, ridx)
    assert rel_err_rows(y, ref) < TOL


def _layer_case(rng, H, I, E, K, svh_scale, rates=None):
    experts = []
    for e in range(E):
        k = K if rates is None else float(rates[e])
        experts.append(synth.expert(rng, H, I, k, svh_scale))
    shared = synth.expert(rng, H, I, K, svh_scale)
    return experts, shared


@pytest.mark.parametrize("limit", [10.0, CLIP])
@pytest.mark.parametrize("rows", [1, 2, 3, 4, 5, 16])
@pytest.mark.parametrize("K", [2, 3, 4, 5, 1.5, 2.5, 3.5])
def test_moe_layer_small(dev, rows, K, limit):
    """Layer parity through the decode GEMV (1-2 rows) and the MFMA tiles (3+ rows); at CLIP the
    SwiGLU limit clips and both clamp orders (routed after SiLU, shared before) are checked."""
    ops = _ops()
    H, I, E, topk = 512, 256, 24, 4
    rng = np.random.default_rng(int(1000 * rows + 2 * K))
    experts, shared = _layer_case(rng, H, I, E, K, 1 / np.sqrt(H))
    x = synth.activations_bf16(rng, rows, H)
    logits = synth.logits_skewed(rng, rows, E, hot=1, warm=3)
    ref, ridx, rw, rrw = coop.moe_layer(x, logits, experts, shared, topk, limit)

    de = DeviceExperts(experts, dev)
    ds = DeviceExperts([shared], dev)
    ws = ops.MoeWorkspace(dev, rows_max=16, hidden=H, inter=I, topk=topk, n_local=E, has_shared=True)
    xt = to_dev(x, dev).to(torch.bfloat16)
    sel = torch.empty(rows, topk, dtype=torch.int64, device=dev)
    w = torch.empty(rows, topk, dtype=torch.float32, device=dev)
    out = torch.empty(rows, H, dtype=torch.float32, device=dev)
    ops.moe_forward(ws, xt, de.table, out, limit=limit, bits=K, logits=to_dev(logits, dev), sel=sel, weights=w,
                    shared_ptrs=ds.ptrs(0), shared_bits=K)
    torch.cuda.synchronize()
    assert np.array_equal(sel.cpu().numpy(), ridx)
    assert int(ws.flags().cpu()[0]) == 0
    y = out.cpu().numpy()
    assert rel_err_rows(y, ref) < TOL
    runs = ws.runs().cpu().numpy()
    assert np.array_equal(runs, coop.reference_table(ridx, rrw, capacity=16))
    if limit == CLIP:
        _assert_clamp_parity(y, clamp_variants(lambda: coop.moe_layer(x, logits, experts, shared, topk, limit)[0]))


@pytest.mark.parametrize("rows", [1, 2])
def test_moe_layer_wide_intermediate(dev, rows):
    """An intermediate width past DSv3's (I = 2560, 20 activation chunks per row, 5 per k-split
    of the down GEMV at the defaults) through the decode GEMV path, against the oracle."""
    ops = _ops()
    H, I, E, topk, limit, K = 512, 2560, 12, 4, 10.0, 4
    rng = np.random.default_rng(77 + rows)
    experts, shared = _layer_case(rng, H, I, E, K, 1 / np.sqrt(H))
    x = synth.activations_bf16(rng, rows, H)
    logits = synth.logits_skewed(rng, rows, E, hot=1, warm=3)
    ref, ridx, _, _ = coop.moe_layer(x, logits, experts, shared, topk, limit)
    de = DeviceExperts(experts, dev)
    ds = DeviceExperts([shared], dev)
    ws = ops.MoeWorkspace(dev, rows_max=rows, hidden=H, inter=I, topk=topk, n_local=E, has_shared=True)
    sel = torch.empty(rows, topk, dtype=torch.int64, device=dev)
    w = torch.empty(rows, topk, dtype=torch.float32, device=dev)
    out = torch.empty(rows, H, dtype=torch.float32, device=dev)
    ops.moe_forward(ws, to_dev(x, dev).to(torch.bfloat16), de.table, out, limit=limit, bits=K,
                    logits=to_dev(logits, dev), sel=sel, weights=w, shared_ptrs=ds.ptrs(0), shared_bits=K)
    torch.cuda.synchronize()
    assert np.array_equal(sel.cpu().numpy(), ridx)
    assert int(ws.flags().cpu()[0]) == 0
    assert rel_err_rows(out.cpu().numpy(), ref) < TOL


_DSV3_CASES = {}


def _dsv3_case(rows):
    """Seeded DSv3-shape inputs and the touched experts (cached per rows)."""
    if rows not in _DSV3_CASES:
        H, I, E, topk, K = 7168, 2048, 256, 8, 4
        rng = np.random.default_rng(42 + rows)
        x = synth.activations_bf16(rng, rows, H)
        logits = synth.logits_plain(rng, rows, E) if rows == 1 else synth.logits_skewed(rng, rows, E)
        ridx, rwt = coop.route(logits, topk)
        used = sorted(set(int(v) for v in ridx.reshape(-1)))
        experts = {e: synth.expert(rng, H, I, K, 1 / np.sqrt(H)) for e in used}
        shared = synth.expert(rng, H, I, K, 1 / np.sqrt(H))
        _DSV3_CASES[rows] = (x, logits, ridx, used, experts, shared, {})
    return _DSV3_CASES[rows]


def _dsv3_ref(rows, limit):
    x, logits, _, _, experts, shared, refs = _dsv3_case(rows)
    if limit not in refs:
        compute = lambda: coop.moe_layer(x, logits, experts, shared, 8, limit)[0]
        refs[limit] = clamp_variants(compute) if limit == CLIP else {"ref": compute()}
    return refs[limit]


@pytest.mark.parametrize("rows", [1, 16])
@pytest.mark.parametrize("ks,limit", [((0, 0), 10.0), ((32, 16), 10.0), ((3, 5), 10.0), ((0, 0), CLIP)])
def test_moe_layer_dsv3_shape(dev, rows, ks, limit):
    """DeepSeek-V3 shape (H=7168, I=2048, 256 routed + 1 shared, top-8, 4 bpw), oracle on the
    touched experts only; automatic k-splits, and requested ones above and below the split that
    fills the GPU once (every split's partials must be written and summed); at CLIP the SwiGLU
    limit clips in both the routed and the shared expert."""
    ops = _ops()
    H, I, E, topk, K = 7168, 2048, 256, 8, 4
    x, logits, ridx, used, experts, shared, _ = _dsv3_case(rows)
    variants = _dsv3_ref(rows, limit)

    # Device table: touched experts at their indices, a dummy expert everywhere else.
    dummy = synth.expert(np.random.default_rng(0), H, I, K)
    de = DeviceExperts([experts[e] for e in used] + [dummy], dev)
    table = torch.empty(9, E, dtype=torch.int64)
    cols = {e: i for i, e in enumerate(used)}
    host = de.table.cpu()
    for e in range(E):
        table[:, e] = host[:, cols.get(e, len(used))]
    table = table.to(dev)
    ds = DeviceExperts([shared], dev)
    ws = ops.MoeWorkspace(dev, rows_max=rows, hidden=H, inter=I, topk=topk, n_local=E, has_shared=True,
                          ksplit_gu=ks[0], ksplit_down=ks[1])
    # stale partials from an earlier call must not leak into this one
    ws.buffer.fill_(0x7f)
    ws.clear_flags()
    sel = torch.empty(rows, topk, dtype=torch.int64, device=dev)
    w = torch.empty(rows, topk, dtype=torch.float32, device=dev)
    out = torch.empty(rows, H, dtype=torch.float32, device=dev)
    ops.moe_forward(ws, to_dev(x, dev).to(torch.bfloat16), table, out, limit=limit, bits=K,
                    logits=to_dev(logits, dev), sel=sel, weights=w, shared_ptrs=ds.ptrs(0), shared_bits=K)
    torch.cuda.synchronize()
    assert np.array_equal(sel.cpu().numpy(), ridx)
    y = out.cpu().numpy()
    assert rel_err_rows(y, variants["ref"]) < TOL
    if limit == CLIP:
        _assert_clamp_parity(y, variants)


@pytest.mark.parametrize("rate_set", [(2, 3, 4, 5), (1.5, 2.5, 3.5, 4)])
def test_moe_mixed_rates_and_given_routes(dev, rate_set):
    ops = _ops()
    H, I, E, topk, limit = 256, 256, 10, 3, 0.0
    rng = np.random.default_rng(5 + len(rate_set) + int(2 * rate_set[0]))
    rates = synth.mixed_rates(rng, E, rate_set)
    experts, _ = _layer_case(rng, H, I, E, 4, 1 / np.sqrt(H), rates)
    rows = 7
    x = rng.standard_normal((rows, H)).astype(np.float16)
    sel = np.stack([rng.choice(E, size=topk, replace=False) for _ in range(rows)]).astype(np.int64)
    rw = rng.uniform(0.1, 1.0, size=(rows, topk)).astype(np.float16)
    rw[2, 1] = 0                                                  # one inactive slot
    ref = coop.moe_routed(x, sel, rw, experts, limit)
    de = DeviceExperts(experts, dev)
    ws = ops.MoeWorkspace(dev, rows_max=8, hidden=H, inter=I, topk=topk, n_local=E, has_shared=False)
    out = torch.empty(rows, H, dtype=torch.float32, device=dev)
    ops.moe_forward(ws, to_dev(x, dev), de.table, out, limit=limit, k2_per_expert=de.k2,
                    sel=to_dev(sel, dev), rw=to_dev(rw, dev))
    torch.cuda.synchronize()
    assert rel_err_rows(out.cpu().numpy(), ref) < TOL


@pytest.mark.parametrize("rows", [1, 2, 3])
def test_moe_given_routes_repeating_an_expert(dev, rows):
    """Given routes may name one expert in several slots of a token (the runner passes them
    through); every slot is its own product, so an expert's chunk holds more rows than there are
    tokens: the one- and two-row decode GEMVs walk them in groups, the MFMA tiles take them as
    rows."""
    ops = _ops()
    H, I, E, topk, limit = 256, 256, 5, 8, 0.0
    rng = np.random.default_rng(300 + rows)
    experts, _ = _layer_case(rng, H, I, E, 4, 1 / np.sqrt(H))
    x = rng.standard_normal((rows, H)).astype(np.float16)
    sel = rng.integers(0, E, size=(rows, topk)).astype(np.int64)      # 8 picks of 5 experts
    sel[0, :4] = 2                                                    # one expert in 4 slots
    rw = rng.uniform(0.1, 1.0, size=(rows, topk)).astype(np.float16)
    ref = coop.moe_routed(x, sel, rw, experts, limit)
    de = DeviceExperts(experts, dev)
    ws = ops.MoeWorkspace(dev, rows_max=rows, hidden=H, inter=I, topk=topk, n_local=E, has_shared=False)
    out = torch.empty(rows, H, dtype=torch.float32, device=dev)
    ops.moe_forward(ws, to_dev(x, dev), de.table, out, limit=limit, bits=4, sel=to_dev(sel, dev), rw=to_dev(rw, dev))
    torch.cuda.synchronize()
    assert int(ws.flags().cpu()[0]) == 0
    assert rel_err_rows(out.cpu().numpy(), ref) < TOL


@pytest.mark.parametrize("rows,pattern", [(3, "all_one"), (16, "hot_twice"), (2, "all_one"), (20, "hot_twice"),
                                          (17, "all_one"), (72, "hot_twice")])
def test_moe_repeated_expert_fills_many_tiles(dev, rows, pattern):
    """Given routes repeating an expert inside tokens put more slots on one expert than a 16-row
    MFMA tile holds: T=3 with all 24 slots on one expert, T=16 with one expert twice in every
    token (32 slots), against the oracle over a workspace filled with garbage first (a tile
    whose partials were never written would read it). Past 16 tokens one expert spans tiles of
    both size classes, which run gate/up, activation and down on different streams: T=17 puts
    136 slots on one expert (tiles of 64, 64 and 8 rows), T=72 144 slots on one (64, 64, 16)
    and the shared expert 72 rows (64 and 8)."""
    ops = _ops()
    H, I, E, topk, limit = 256, 256, 6, 8, CLIP
    rng = np.random.default_rng(400 + rows)
    experts, shared = _layer_case(rng, H, I, E, 4, 1 / np.sqrt(H))
    x = rng.standard_normal((rows, H)).astype(np.float16)
    sel = rng.integers(0, E, size=(rows, topk)).astype(np.int64)
    if pattern == "all_one":
        sel[:] = 2
    else:
        sel[:, 0] = sel[:, 5] = 4
    rw = rng.uniform(0.1, 1.0, size=(rows, topk)).astype(np.float16)
    ref = coop.moe_routed(x, sel, rw, experts, limit)
    ref = (ref + coop.shared_expert(x, shared, limit)).astype(np.float32)
    de, ds = DeviceExperts(experts, dev), DeviceExperts([shared], dev)
    ws = ops.MoeWorkspace(dev, rows_max=rows, hidden=H, inter=I, topk=topk, n_local=E, has_shared=True)
    ws.buffer.fill_(0x7f)
    ws.clear_flags()
    out = torch.empty(rows, H, dtype=torch.float32, device=dev)
    ops.moe_forward(ws, to_dev(x, dev), de.table, out, limit=limit, bits=4, sel=to_dev(sel, dev),
                    rw=to_dev(rw, dev), shared_ptrs=ds.ptrs(0), shared_bits=4)
    torch.cuda.synchronize()
    assert int(ws.flags().cpu()[0]) == 0
    assert rel_err_rows(out.cpu().numpy(), ref) < TOL


@pytest.mark.parametrize("rows", [1, 4])
def test_moe_bf16_x_rounds_to_fp16(dev, rows):
    """The reference casts the activations to fp16 before routing and the experts
    (model.py:455): bf16 values past the fp16 range become inf, and values in the fp16 subnormal
    range lose precision or flush. Row 0 holds 70000 (inf in fp16: that row's output is all
    non-finite, as the oracle's); the other rows hold subnormal-range values, including 2e-8,
    which rounds to zero (their effect on a layer output is below the tolerance; the router
    test checks their rounding against fp32-tight logits)."""
    ops = _ops()
    H, I, E, topk, limit, K = 512, 256, 16, 4, 10.0, 4
    rng = np.random.default_rng(500 + rows)
    experts, shared = _layer_case(rng, H, I, E, K, 1 / np.sqrt(H))
    x = synth.activations_bf16(rng, rows, H)
    x[0, 17] = 70000.0
    tiny = np.array([3.0e-5, -1.1e-6, 2.0e-8, 6.0e-7, -4.4e-5], np.float32)
    for r in range(1, rows):
        x[r, 5 * r:5 * r + 5] = tiny
    x = coop.round_bf16(x)
    assert np.isinf(x.astype(np.float16)[0, 17]) and (x.astype(np.float16)[1:, :] == 0).sum() >= rows - 1
    logits = synth.logits_skewed(rng, rows, E, hot=1, warm=3)
    ref, ridx, _, _ = coop.moe_layer(x, logits, experts, shared, topk, limit)
    de, ds = DeviceExperts(experts, dev), DeviceExperts([shared], dev)
    ws = ops.MoeWorkspace(dev, rows_max=rows, hidden=H, inter=I, topk=topk, n_local=E, has_shared=True)
    sel = torch.empty(rows, topk, dtype=torch.int64, device=dev)
    w = torch.empty(rows, topk, dtype=torch.float32, device=dev)
    out = torch.empty(rows, H, dtype=torch.float32, device=dev)
    ops.moe_forward(ws, to_dev(x, dev).to(torch.bfloat16), de.table, out, limit=limit, bits=K,
                    logits=to_dev(logits, dev), sel=sel, weights=w, shared_ptrs=ds.ptrs(0), shared_bits=K)
    torch.cuda.synchronize()
    assert np.array_equal(sel.cpu().numpy(), ridx)
    y = out.cpu().numpy()
    assert not np.isfinite(ref[0]).any() and not np.isfinite(y[0]).any()
    if rows > 1:
        assert np.isfinite(y[1:]).all()
        assert rel_err_rows(y[1:], ref[1:]) < TOL


@pytest.mark.parametrize("rows", [4, 40])
def test_rotated_inputs_bit_exact(dev, rows):
    """The input rotation on its own (K.cuh:613-629): every active routed slot's and every
    shared row's gate and up inputs fp16(H128(fp16(x) * suh)) in the workspace equal the oracle's
    bit for bit (same fp32 butterfly order, same roundings), with bf16 activations that include
    fp16-subnormal-range values. 4 rows rotate in the small prepare, 40 in the rotation kernel of
    the prefill path; zero routing weights leave some slots inactive."""
    ops = _ops()
    H, I, E, topk, K = 512, 256, 16, 4, 4
    rng = np.random.default_rng(700 + rows)
    experts, shared = _layer_case(rng, H, I, E, K, 1 / np.sqrt(H))
    x = synth.activations_bf16(rng, rows, H)
    x[:, 3] = np.array([3.0e-5, -1.1e-6, 6.0e-7, -4.4e-5] * rows, np.float32)[:rows]
    x = coop.round_bf16(x)
    sel = rng.integers(0, E, size=(rows, topk)).astype(np.int64)
    rw = rng.uniform(0.1, 1.0, size=(rows, topk)).astype(np.float16)
    rw[rng.random((rows, topk)) < 0.2] = 0
    de, ds = DeviceExperts(experts, dev), DeviceExperts([shared], dev)
    ws = ops.MoeWorkspace(dev, rows_max=rows, hidden=H, inter=I, topk=topk, n_local=E, has_shared=True)
    out = torch.empty(rows, H, dtype=torch.float32, device=dev)
    ops.moe_forward(ws, to_dev(x, dev).to(torch.bfloat16), de.table, out, limit=10.0, bits=K,
                    sel=to_dev(sel, dev), rw=to_dev(rw, dev), shared_ptrs=ds.ptrs(0), shared_bits=K)
    torch.cuda.synchronize()
    assert int(ws.flags().cpu()[0]) == 0
    xr = ws.rotated().cpu().numpy()
    x16 = x.astype(np.float16)
    checked = 0
    for pi, p in enumerate(("g", "u")):
        for r in range(rows):
            for k in range(topk):
                if rw[r, k] == 0:
                    continue
                ref = coop.rotate_input(x16[r], experts[sel[r, k]].suh(p))
                assert np.array_equal(xr[pi, r * topk + k].view(np.uint16), ref.view(np.uint16)), (p, r, k)
                checked += 1
            ref = coop.rotate_input(x16[r], shared.suh(p))
            assert np.array_equal(xr[pi, rows * topk + r].view(np.uint16), ref.view(np.uint16)), (p, "shared", r)
    assert checked > rows * topk


def test_moe_out_of_range_expert_sets_flag(dev):
    ops = _ops()
    H, I, E, topk = 256, 128, 8, 2
    rng = np.random.default_rng(9)
    experts, _ = _layer_case(rng, H, I, E, 4, 1 / np.sqrt(H))
    de = DeviceExperts(experts, dev)
    ws = ops.MoeWorkspace(dev, rows_max=2, hidden=H, inter=I, topk=topk, n_local=E, has_shared=False)
    x = rng.standard_normal((2, H)).astype(np.float16)
    sel = np.array([[1, 99], [2, 3]], dtype=np.int64)              # 99 is outside the table
    rw = np.array([[0.5, 0.5], [0.5, 0.5]], dtype=np.float16)
    out = torch.empty(2, H, dtype=torch.float32, device=dev)
    ops.moe_forward(ws, to_dev(x, dev), de.table, out, limit=0.0, bits=4, sel=to_dev(sel, dev), rw=to_dev(rw, dev))
    torch.cuda.synchronize()
    assert int(ws.flags().cpu()[0]) & 1
    rw2 = rw.copy()
    rw2[0, 1] = 0                                                  # the flagged slot is dropped
    ref = coop.moe_routed(x, np.where(sel < E, sel, 0), rw2, experts, 0.0)
    assert rel_err_rows(out.cpu().numpy(), ref) < TOL
