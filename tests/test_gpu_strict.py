"""Strict batch mode on the GPU (the reference's DS41_STRICT_BATCH, runtime/ds41/moe_coop.py:17-22:
"keep target and verification arithmetic identical"): with ``strict_rows`` set, a token's routed +
shared output, routes and weights are bit-identical whether it runs alone or inside a call of
2..strict_rows tokens, at the DeepSeek-V3 shape and on reduced shapes that cover mixed and
separate down rates, the gated shared expert, given routes that repeat an expert within a token, an
expert range, fp32 and fp16 given weights, and column-group counts that are and are not a multiple
of the workgroup's four waves. Every strict output is also held to the oracle's tolerance. The
fast (automatic) geometry is shown to change a row's bits across batch sizes, so the bit-equality
checks have teeth. ELinear in strict dense mode keeps a row's bits at 1, 17 and 64 rows."""
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


def _same_bits(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


def _dsv3_table(dev, used, experts):
    """[9, 256] table with the touched experts at their indices, a dummy expert elsewhere."""
    H, I, E, K = 7168, 2048, 256, 4
    dummy = synth.expert(np.random.default_rng(0), H, I, K)
    de = DeviceExperts([experts[e] for e in used] + [dummy], dev)
    table = torch.empty(9, E, dtype=torch.int64)
    cols = {e: i for i, e in enumerate(used)}
    host = de.table.cpu()
    for e in range(E):
        table[:, e] = host[:, cols.get(e, len(used))]
    return de, table.to(dev)


def test_strict_dsv3_rows_bit_identical_across_batch_sizes(dev):
    """DSv3 shape (H=7168, I=2048, 256 routed + 1 shared, top-8, 4 bpw), 16 tokens with skewed
    routing (hot experts shared by several tokens, so chunks hold several rows): every token's
    output in calls of T = 2, 3, 8 and 16 tokens (two different row windows each) equals its
    output alone, bit for bit, and the oracle within the tolerance."""
    from tests.test_gpu_parity import _dsv3_case, _dsv3_ref
    ops = _ops()
    H, I, E, topk, K, rows = 7168, 2048, 256, 8, 4, 16
    x, logits, ridx, used, experts, shared, _ = _dsv3_case(rows)
    ref = _dsv3_ref(rows, 10.0)["ref"]
    de, table = _dsv3_table(dev, used, experts)
    ds = DeviceExperts([shared], dev)
    xd = to_dev(x, dev).to(torch.bfloat16)
    zd = to_dev(logits, dev)

    def run(ws, r0, T):
        sel = torch.empty(T, topk, dtype=torch.int64, device=dev)
        w = torch.empty(T, topk, dtype=torch.float32, device=dev)
        out = torch.empty(T, H, dtype=torch.float32, device=dev)
        ops.moe_forward(ws, xd[r0:r0 + T], table, out, limit=10.0, bits=K, logits=zd[r0:r0 + T], sel=sel,
                        weights=w, shared_ptrs=ds.ptrs(0), shared_bits=K)
        torch.cuda.synchronize()
        return out.cpu().numpy(), sel.cpu().numpy(), w.cpu().numpy()

    ws = ops.MoeWorkspace(dev, rows_max=rows, hidden=H, inter=I, topk=topk, n_local=E, has_shared=True,
                          strict_rows=rows)
    ws.buffer.fill_(0x7f)                      # no stale partials may leak into a call
    ws.clear_flags()
    alone = [run(ws, r, 1) for r in range(rows)]
    y1 = np.concatenate([a[0] for a in alone])
    assert rel_err_rows(y1, ref) < TOL
    assert np.array_equal(np.concatenate([a[1] for a in alone]), ridx)
    for T in (2, 3, 8, 16):
        for r0 in sorted({0, rows - T}):
            y, sel, w = run(ws, r0, T)
            for i in range(T):
                assert _same_bits(y[i], alone[r0 + i][0][0]), (T, r0, i)
                assert np.array_equal(sel[i], alone[r0 + i][1][0]) and _same_bits(w[i], alone[r0 + i][2][0])
    assert int(ws.flags().cpu()[0]) == 0
    # teeth: the automatic geometry gives the 16-token call other bits (MFMA tiles, other splits)
    fast = ops.MoeWorkspace(dev, rows_max=rows, hidden=H, inter=I, topk=topk, n_local=E, has_shared=True)
    y16 = run(fast, 0, 16)[0]
    assert rel_err_rows(y16, ref) < TOL
    assert not _same_bits(y16, y1)


def _small_case(rng, H, I, E, rates=None, down_rates=None, shared_down=None):
    experts = []
    for e in range(E):
        K = float(rates[e]) if rates is not None else 4.0
        Kd = float(down_rates[e]) if down_rates is not None else None
        experts.append(synth.expert(rng, H, I, K, 1 / np.sqrt(H), K_down=Kd))
    shared = synth.expert(rng, H, I, 3.0, 1 / np.sqrt(H), K_down=shared_down)
    return experts, shared


@pytest.mark.parametrize("H, I", [(256, 512), (256, 384), (512, 512)])
@pytest.mark.parametrize("case", ["routed", "mixed_gated", "given_repeats", "other_rates"])
def test_strict_small_shapes_bit_identical(dev, H, I, case):
    """Reduced shapes, up to 32 tokens (256 slots, the strict bound): every row of calls of 2, 3, 5,
    8, 13, 20 and 32 tokens equals the row alone, bit for bit, and the oracle within the tolerance.
    I = 384 (3 column groups of gate/up) takes the 2-row-pass kernel, I = 512 the 8-row one. At
    H = I = 512 (four column groups of each) calls of more than 8 tokens pair each expert's 8-row
    chunks in gate/up and down (up to 16 rows per pass; the expert picked twice by every token in
    given_repeats has 64 slots, four pairs), and down runs the workgroup-staged kernel from 3 tokens.
    mixed_gated and other_rates together run every gate/up and down rate of the decode path."""
    ops = _ops()
    E, topk, rows = 24, 8, 32
    rng = np.random.default_rng({"routed": 1, "mixed_gated": 2, "given_repeats": 3, "other_rates": 4}[case] * 100 + I
                                + (H - 256))
    kw, ref_kw = {}, {}
    x = synth.activations_bf16(rng, rows, H)
    if case == "other_rates":
        # the rates mixed_gated leaves out: gate/up 1.5, 3.5 and 5 bpw, down 1.5, 2, 2.5 and 3.5
        rates = synth.mixed_rates(rng, E, (1.5, 3.5, 5))
        drates = synth.mixed_rates(rng, E, (1.5, 2, 2.5, 3.5))
        experts, shared = _small_case(rng, H, I, E, rates, drates, shared_down=2.5)
        de, ds = DeviceExperts(experts, dev), DeviceExperts([shared], dev)
        kw = dict(k2_per_expert=de.k2, k2_down_per_expert=de.k2_down, shared_bits_down=2.5)
    elif case == "mixed_gated":
        rates = synth.mixed_rates(rng, E, (2, 2.5, 3, 4))
        drates = synth.mixed_rates(rng, E, (3, 4, 5))
        experts, shared = _small_case(rng, H, I, E, rates, drates, shared_down=4.0)
        gate = (rng.standard_normal(H) * 0.05).astype(np.float16)
        de, ds = DeviceExperts(experts, dev), DeviceExperts([shared], dev)
        kw = dict(k2_per_expert=de.k2, k2_down_per_expert=de.k2_down, shared_bits_down=4.0,
                  shared_gate_w=to_dev(gate, dev))
        ref_kw = dict(shared_gate_w=gate)
    else:
        experts, shared = _small_case(rng, H, I, E)
        de, ds = DeviceExperts(experts, dev), DeviceExperts([shared], dev)
        kw = dict(bits=4.0)
    if case == "given_repeats":
        # given routes: expert 5 (local 3) picked twice by every token, expert range [2, 26) over
        # 24 local experts, fp32 weights with some zeros; expert 5's 64 slots form full 8-row chunks
        sel = rng.integers(2, 26, size=(rows, topk)).astype(np.int64)
        sel[:, 1] = 5
        sel[:, 6] = 5
        sel[::5, 2] = 40                                     # outside the range: inactive
        w = rng.uniform(0.05, 1.0, size=(rows, topk)).astype(np.float32)
        w[::7, 4] = 0.0
        rw = w.astype(np.float16)
        ref_y = coop.moe_routed(x.astype(np.float32).astype(np.float16), sel, rw, dict(enumerate(experts)), 10.0,
                                min_expert=2, max_expert=26)
        ref_y = (ref_y + coop.shared_expert(x.astype(np.float32).astype(np.float16), shared, 10.0)).astype(np.float32)
        sd, wd = to_dev(sel, dev), to_dev(w, dev)
        route = lambda r0, T: dict(sel=sd[r0:r0 + T].contiguous(), weights=wd[r0:r0 + T].contiguous(),
                                   min_expert=2, max_expert=26)
    else:
        logits = synth.logits_skewed(rng, rows, E)
        ref_y = coop.moe_layer(x, logits, experts, shared, topk, 10.0, **ref_kw)[0]
        zd = to_dev(logits, dev)
        route = lambda r0, T: dict(logits=zd[r0:r0 + T], sel=torch.empty(T, topk, dtype=torch.int64, device=dev),
                                   weights=torch.empty(T, topk, dtype=torch.float32, device=dev))
    xd = to_dev(x, dev).to(torch.bfloat16)
    ws = ops.MoeWorkspace(dev, rows_max=rows, hidden=H, inter=I, topk=topk, n_local=E, has_shared=True,
                          strict_rows=rows)
    ws.buffer.fill_(0x7f)
    ws.clear_flags()

    def run(r0, T):
        out = torch.empty(T, H, dtype=torch.float32, device=dev)
        ops.moe_forward(ws, xd[r0:r0 + T], de.table, out, limit=10.0, shared_ptrs=ds.ptrs(0), shared_bits=3.0,
                        **route(r0, T), **kw)
        torch.cuda.synchronize()
        return out.cpu().numpy()

    y1 = np.concatenate([run(r, 1) for r in range(rows)])
    assert rel_err_rows(y1, ref_y) < TOL
    for T in (2, 3, 5, 8, 13, 20, 32):
        for r0 in sorted({0, rows - T}):
            y = run(r0, T)
            assert _same_bits(y, y1[r0:r0 + T]), (T, r0)
    flags = int(ws.flags().cpu()[0])
    assert flags == 0


def test_strict_calls_above_the_bound_take_the_fast_path(dev):
    """strict_rows = 4: calls of up to 4 rows keep the one-row bits, a 12-row call takes the
    automatic geometry (MFMA tiles) and stays within the tolerance."""
    ops = _ops()
    H, I, E, topk = 256, 512, 16, 4
    rng = np.random.default_rng(77)
    experts, shared = _small_case(rng, H, I, E)
    de, ds = DeviceExperts(experts, dev), DeviceExperts([shared], dev)
    x = synth.activations_bf16(rng, 12, H)
    logits = synth.logits_plain(rng, 12, E)
    ref = coop.moe_layer(x, logits, experts, shared, topk, 10.0)[0]
    ws = ops.MoeWorkspace(dev, rows_max=12, hidden=H, inter=I, topk=topk, n_local=E, has_shared=True, strict_rows=4)
    xd, zd = to_dev(x, dev).to(torch.bfloat16), to_dev(logits, dev)

    def run(r0, T):
        out = torch.empty(T, H, dtype=torch.float32, device=dev)
        sel = torch.empty(T, topk, dtype=torch.int64, device=dev)
        w = torch.empty(T, topk, dtype=torch.float32, device=dev)
        ops.moe_forward(ws, xd[r0:r0 + T], de.table, out, limit=10.0, bits=4.0, logits=zd[r0:r0 + T], sel=sel,
                        weights=w, shared_ptrs=ds.ptrs(0), shared_bits=3.0)
        torch.cuda.synchronize()
        return out.cpu().numpy()

    y1 = np.concatenate([run(r, 1) for r in range(12)])
    assert _same_bits(run(4, 4), y1[4:8])
    y12 = run(0, 12)
    assert rel_err_rows(y12, ref) < TOL and rel_err_rows(y1, ref) < TOL


def test_strict_router_front_no_shared(dev):
    """Strict mode through the router front (logits from the fp32 gate weight inside the call),
    sqrt-softplus scores with a selection bias, and no shared expert: every row of calls of 2, 6
    and 11 tokens equals the row alone, bit for bit (routes, weights and output), and the oracle's
    layer on the kernel's own logits within the tolerance."""
    ops = _ops()
    H, I, E, topk, rows = 512, 512, 24, 6, 11
    rng = np.random.default_rng(79)
    experts, _ = _small_case(rng, H, I, E)
    de = DeviceExperts(experts, dev)
    x = synth.activations_bf16(rng, rows, H)
    gate_w = (rng.standard_normal((E, H)) / np.sqrt(H)).astype(np.float32)
    bias = (0.1 * rng.standard_normal(E)).astype(np.float32)
    ws = ops.MoeWorkspace(dev, rows_max=rows, hidden=H, inter=I, topk=topk, n_local=E, has_shared=False,
                          strict_rows=rows)
    xd, gd, bd = to_dev(x, dev).to(torch.bfloat16), to_dev(gate_w, dev), to_dev(bias, dev)

    def run(r0, T):
        out = torch.empty(T, H, dtype=torch.float32, device=dev)
        sel = torch.empty(T, topk, dtype=torch.int64, device=dev)
        w = torch.empty(T, topk, dtype=torch.float32, device=dev)
        ops.moe_forward(ws, xd[r0:r0 + T], de.table, out, limit=10.0, bits=4.0, gate_w=gd, sel=sel, weights=w,
                        score_fn="sqrt_softplus", sel_bias=bd)
        torch.cuda.synchronize()
        z = ws.logits(T, E).cpu().numpy().copy()
        return out.cpu().numpy(), sel.cpu().numpy(), w.cpu().numpy(), z

    alone = [run(r, 1) for r in range(rows)]
    z1 = np.concatenate([a[3] for a in alone])
    ref = coop.moe_layer(x, z1, experts, None, topk, 10.0, score_fn="sqrt_softplus", sel_bias=bias)[0]
    y1 = np.concatenate([a[0] for a in alone])
    assert rel_err_rows(y1, ref) < TOL
    for T in (2, 6, 11):
        for r0 in sorted({0, rows - T}):
            y, sel, w, z = run(r0, T)
            assert _same_bits(z, z1[r0:r0 + T]), (T, r0)
            for i in range(T):
                a = alone[r0 + i]
                assert _same_bits(y[i], a[0][0]) and np.array_equal(sel[i], a[1][0]) and _same_bits(w[i], a[2][0])
    assert int(ws.flags().cpu()[0]) == 0


@pytest.mark.parametrize("H, T", [(256, 8), (512, 16)])
def test_strict_graph_replays(dev, H, T):
    """A strict 8-token call (wide prepare, 8-row kernels) and a 16-token one at H = I = 512 (paired
    chunks, workgroup-staged down) captured into a graph: three replays, with eager calls of other
    sizes in between, each bit-identical to the eager call."""
    ops = _ops()
    I, E, topk = 512, 16, 8
    rng = np.random.default_rng(78 + T)
    experts, shared = _small_case(rng, H, I, E)
    de, ds = DeviceExperts(experts, dev), DeviceExperts([shared], dev)
    x = to_dev(synth.activations_bf16(rng, T, H), dev).to(torch.bfloat16)
    z = to_dev(synth.logits_skewed(rng, T, E), dev)
    ws = ops.MoeWorkspace(dev, rows_max=T, hidden=H, inter=I, topk=topk, n_local=E, has_shared=True, strict_rows=T)
    sel = torch.empty(T, topk, dtype=torch.int64, device=dev)
    w = torch.empty(T, topk, dtype=torch.float32, device=dev)
    out = torch.empty(T, H, dtype=torch.float32, device=dev)
    call = lambda n: ops.moe_forward(ws, x[:n], de.table, out[:n], limit=10.0, bits=4.0, logits=z[:n], sel=sel[:n],
                                     weights=w[:n], shared_ptrs=ds.ptrs(0), shared_bits=3.0)
    call(T)
    torch.cuda.synchronize()
    eager = out.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call(T)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(T)
    for n in (3, 5, 1, T - 2):
        out.zero_()
        call(n)                                          # eager work of another size in between
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), eager.view(torch.int32))


def test_elinear_strict_dense_rows(dev):
    """Strict dense mode: with the verification bound at 64 rows a row gives the bits it gets alone
    in calls of 17 and 64 rows (16-row decode GEMV calls); with strict mode off the 17-row call takes
    the MFMA tiles and the row's bits change."""
    from eva_amd import linear, verification
    rng = np.random.default_rng(66)
    tr, suh, svh = synth.projection(rng, 512, 384, 4, svh_scale=1 / np.sqrt(512))
    args = (torch.from_numpy(suh), torch.from_numpy(svh), torch.from_numpy(tr), None)
    x = rng.standard_normal((64, 512)).astype(np.float16)
    ref = coop.exl3_linear(x, tr, suh, svh, 4)
    old = verification._MAX_ROWS
    verification._MAX_ROWS = 64
    try:
        lin = linear.build_linear(*args, device=dev, strict=True)
        alone = np.concatenate([lin.forward(to_dev(x[i:i + 1], dev)).cpu().numpy() for i in range(64)])
        y17 = lin.forward(to_dev(x[:17], dev)).cpu().numpy()
        y64 = lin.forward(to_dev(x, dev)).cpu().numpy()
        assert np.array_equal(y17.view(np.uint16), alone[:17].view(np.uint16))
        assert np.array_equal(y64.view(np.uint16), alone.view(np.uint16))
        assert rel_err_rows(y64.astype(np.float32), ref.astype(np.float32)) < TOL
        fast = linear.build_linear(*args, device=dev, strict=False)
        f17 = fast.forward(to_dev(x[:17], dev)).cpu().numpy()
        assert rel_err_rows(f17.astype(np.float32), ref[:17].astype(np.float32)) < TOL
        assert not np.array_equal(f17.view(np.uint16), alone[:17].view(np.uint16))
    finally:
        verification._MAX_ROWS = old
