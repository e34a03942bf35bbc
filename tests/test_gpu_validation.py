"""moe_forward refuses malformed arguments with ValueError before any launch.

The C ABI receives bare device pointers and sizes, so a tensor of the wrong shape, dtype or
device would make the kernels read or write out of bounds; eva_amd.ops.moe_forward checks every
tensor against the workspace's shape first. Device tensors are needed to reach those checks, so
these tests are marked gpu, but none of them launches a kernel.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

H, I, E, TOPK, ROWS = 256, 128, 8, 2, 4


@pytest.fixture()
def base(dev):
    from eva_amd import ops
    ws = ops.MoeWorkspace(dev, rows_max=ROWS, hidden=H, inter=I, topk=TOPK, n_local=E, has_shared=False)
    f = lambda *shape, dtype=torch.float32: torch.zeros(*shape, dtype=dtype, device=dev)
    args = dict(x=f(ROWS, H, dtype=torch.float16), tables=f(9, E, dtype=torch.int64), out=f(ROWS, H),
                sel=f(ROWS, TOPK, dtype=torch.int64), weights=f(ROWS, TOPK), logits=f(ROWS, E))
    return ops, ws, args, f


def _call(ops, ws, **kw):
    a = dict(kw)
    x, tables, out = a.pop("x"), a.pop("tables"), a.pop("out")
    return ops.moe_forward(ws, x, tables, out, limit=1.0, bits=a.pop("bits", 4), **a)


@pytest.mark.parametrize("field,make", [
    ("x", lambda f: f(ROWS, H + 128, dtype=torch.float16)),           # wrong hidden
    ("x", lambda f: f(ROWS + 1, H, dtype=torch.float16)),             # more rows than the workspace
    ("x", lambda f: f(ROWS, H)),                                      # fp32 activations
    ("x", lambda f: torch.zeros(ROWS, H, dtype=torch.float16)),      # host tensor
    ("tables", lambda f: f(9, E + 1, dtype=torch.int64)),
    ("tables", lambda f: f(9, E, dtype=torch.int32)),
    ("out", lambda f: f(ROWS - 1, H)),                                # too few rows
    ("out", lambda f: f(ROWS, H - 128)),                              # too narrow
    ("out", lambda f: f(ROWS, H, dtype=torch.float16)),
    ("sel", lambda f: f(ROWS, TOPK + 1, dtype=torch.int64)),
    ("sel", lambda f: f(ROWS - 1, TOPK, dtype=torch.int64)),
    ("sel", lambda f: f(ROWS, TOPK, dtype=torch.int32)),
    ("sel", lambda f: torch.zeros(ROWS, TOPK, dtype=torch.int64)),   # host tensor
    ("weights", lambda f: f(ROWS, TOPK + 1)),
    ("weights", lambda f: f(ROWS, TOPK, dtype=torch.float16)),
    ("weights", lambda f: torch.zeros(ROWS, TOPK)),                   # host tensor
    ("logits", lambda f: f(ROWS - 1, E)),
    ("logits", lambda f: f(ROWS, 1)),                                 # fewer experts than topk
    ("logits", lambda f: f(ROWS, 513)),
    ("logits", lambda f: f(ROWS, E, dtype=torch.float16)),
])
def test_malformed_tensor_rejected(base, field, make):
    ops, ws, args, f = base
    args[field] = make(f)
    with pytest.raises(ValueError):
        _call(ops, ws, **args)


def test_other_malformed_arguments(base):
    ops, ws, args, f = base
    given = {k: v for k, v in args.items() if k != "logits"}
    with pytest.raises(ValueError):                                   # routing needs a weights output
        _call(ops, ws, **{**args, "weights": None})
    with pytest.raises(ValueError):                                   # logits and gate_w together
        _call(ops, ws, **args, gate_w=f(E, H))
    with pytest.raises(ValueError):                                   # gate_w of the wrong width
        _call(ops, ws, **{**given, "gate_w": f(E, H + 128)})
    with pytest.raises(ValueError):                                   # sel_bias of the wrong length
        _call(ops, ws, **args, sel_bias=f(E + 1))
    with pytest.raises(ValueError):                                   # given routes without weights
        _call(ops, ws, **{**given, "weights": None})
    with pytest.raises(ValueError):                                   # rw of the wrong dtype
        _call(ops, ws, **{**given, "weights": None, "rw": f(ROWS, TOPK)})
    with pytest.raises(ValueError):                                   # k2 table of the wrong length
        _call(ops, ws, **given, bits=None, k2_per_expert=f(E - 1, dtype=torch.uint8))
    with pytest.raises(ValueError):                                   # no rate at all
        _call(ops, ws, **given, bits=None)
    with pytest.raises(ValueError):                                   # residual rows differ
        _call(ops, ws, **{**given, "out": None}, residual=f(ROWS - 1, H, dtype=torch.bfloat16))
    with pytest.raises(ValueError):                                   # shared pointers, no shared expert
        _call(ops, ws, **given, shared_ptrs=[0] * 9, shared_bits=4)
    with pytest.raises(ValueError):                                   # wrong number of events
        _call(ops, ws, **given, events=[0] * 4)
    from eva_amd import ops as _ops
    wsh = _ops.MoeWorkspace(args["x"].device, rows_max=ROWS, hidden=H, inter=I, topk=TOPK, n_local=E,
                            has_shared=True)
    with pytest.raises(ValueError):                                   # shared expert missing
        _call(ops, wsh, **given)
    torch.cuda.synchronize()
    assert int(ws.flags().cpu()[0]) == 0                              # nothing ran
