"""The C-ABI library on the host (no GPU): it loads, exports every symbol the header declares,
its structs have the layout the header gives them, and it rejects bad arguments with the
documented error codes before touching a device (the reference's synchronous TORCH_CHECK
validation, runtime/ds41/csrc/moe_coop3072/moe_coop3072.cu:76-124)."""
import ctypes
import os
import re
import subprocess

import pytest

from eva_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "evamx.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(evamx_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = _declared()
    assert len(names) >= 14
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(_lib.EXPORTS)
    assert L.evamx_abi_version() == _lib.ABI_VERSION


def test_struct_layout_matches_header(tmp_path):
    fields = {"evamx_moe_shape": [f for f, _ in _lib.MoeShape._fields_],
              "evamx_moe_args": [f for f, _ in _lib.MoeArgs._fields_]}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "evamx.h"', 'int main(void) {']
    for st, fs in fields.items():
        lines.append(f'printf("{st} size %zu\\n", sizeof({st}));')
        for f in fs:
            lines.append(f'printf("{st} {f} %zu\\n", offsetof({st}, {f}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = {tuple(l.split()[:2]): int(l.split()[2]) for l in out if l}
    for st, cls in (("evamx_moe_shape", _lib.MoeShape), ("evamx_moe_args", _lib.MoeArgs)):
        assert got[(st, "size")] == ctypes.sizeof(cls)
        for f in fields[st]:
            assert got[(st, f)] == getattr(cls, f).offset, (st, f)


def _shape(**kw):
    d = dict(rows_max=16, hidden=7168, inter=2048, topk=8, n_local=256, has_shared=1, ksplit_gu=0, ksplit_down=0,
             strict_rows=0)
    d.update(kw)
    return _lib.MoeShape(*[d[f] for f, _ in _lib.MoeShape._fields_])


def test_workspace_bytes():
    L = _lib.lib()
    sizes = [L.evamx_moe_workspace_bytes(ctypes.byref(_shape(rows_max=r))) for r in (1, 2, 16, 512)]
    assert all(s > 0 and s % 256 == 0 for s in sizes)
    assert sizes == sorted(sizes)
    # DSv3 T=16 scratch is small next to the 2.27 GB of weights the step reads
    assert sizes[2] < 64 << 20
    for bad in (dict(hidden=7100), dict(inter=0), dict(topk=0), dict(topk=33), dict(n_local=513),
                dict(rows_max=0), dict(ksplit_gu=65), dict(rows_max=65536, topk=8), dict(strict_rows=-1),
                dict(strict_rows=65, topk=1), dict(strict_rows=33, topk=8)):
        assert L.evamx_moe_workspace_bytes(ctypes.byref(_shape(**bad))) == 0, bad
        assert L.evamx_last_error()
    assert L.evamx_prepare_routes_workspace_bytes(0, 8) == 0
    # strict mode: room for the decode path's records and one-row splits at every row count up to
    # strict_rows; DSv3 strict verification batches of 16 rows stay far below the weights they read
    for r in (1, 2, 16, 32):
        plain = L.evamx_moe_workspace_bytes(ctypes.byref(_shape(rows_max=r)))
        strict = L.evamx_moe_workspace_bytes(ctypes.byref(_shape(rows_max=r, strict_rows=min(r, 32))))
        assert strict >= plain > 0
    assert L.evamx_moe_workspace_bytes(ctypes.byref(_shape(rows_max=16, strict_rows=16))) < 64 << 20
    assert L.evamx_moe_workspace_bytes(ctypes.byref(_shape(rows_max=512, strict_rows=8))) > 0
    assert L.evamx_exl3_linear_workspace_bytes(1, 2048, 7168) > 2048 * 2


FAKE = 0x10000      # never dereferenced: every case below fails validation first


def _args(**kw):
    a = _lib.MoeArgs()
    a.shape = _shape(rows_max=4, has_shared=0)
    a.rows, a.x, a.x_dtype, a.x_stride = 2, FAKE, _lib.DTYPE_BF16, 7168
    a.sel, a.weights, a.tables, a.bits, a.limit = FAKE, FAKE, FAKE, 4.0, 10.0
    a.out, a.out_stride, a.workspace = FAKE, 7168, FAKE
    a.min_expert, a.max_expert = -1, 0
    a.workspace_bytes = _lib.lib().evamx_moe_workspace_bytes(ctypes.byref(a.shape))
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("bad,msg", [
    (dict(rows=0), "rows"), (dict(rows=5), "rows"), (dict(x=0), "null"), (dict(out=0), "null"),
    (dict(x_dtype=7), "x_dtype"), (dict(x_stride=100), "strides"), (dict(limit=-1.0), "limit"),
    (dict(limit=float("inf")), "limit"), (dict(bits=1.0), "bit rate"), (dict(bits=6.0), "bit rate"), (dict(bits=4.5), "bit rate"),
    (dict(weights=0), "weights"), (dict(min_expert=4, max_expert=4), "range"),
    (dict(logits=FAKE, n_logits=4), "n_logits"), (dict(logits=FAKE, n_logits=256, score_fn=3), "score"),
    (dict(logits=FAKE, gate_w=FAKE, n_logits=256), "not both"), (dict(gate_w=FAKE + 4, n_logits=256), "gate_w"),
    (dict(gate_w=FAKE, n_logits=4), "n_logits"), (dict(gate_w=FAKE, n_logits=256, weights=0), "weights"),
])
def test_forward_rejects_bad_arguments(bad, msg):
    L = _lib.lib()
    a = _args(**bad)
    assert L.evamx_moe_forward(ctypes.byref(a), None) == _lib.EVAMX_EINVAL
    assert msg in L.evamx_last_error().decode()


def test_forward_rejects_short_workspace_and_missing_shared():
    L = _lib.lib()
    a = _args()
    a.workspace_bytes -= 256
    assert L.evamx_moe_forward(ctypes.byref(a), None) == _lib.EVAMX_ENOSPACE
    a = _args()
    a.shape.has_shared = 1
    a.workspace_bytes = L.evamx_moe_workspace_bytes(ctypes.byref(a.shape))
    assert L.evamx_moe_forward(ctypes.byref(a), None) == _lib.EVAMX_EINVAL
    assert "shared" in L.evamx_last_error().decode()


def test_other_entry_points_reject_bad_arguments():
    L = _lib.lib()
    assert L.evamx_exl3_dequant(FAKE, 2048, 7168, 4.25, FAKE, None) == _lib.EVAMX_EINVAL
    assert L.evamx_exl3_dequant(FAKE, 2040, 7168, 4.0, FAKE, None) == _lib.EVAMX_EINVAL
    assert L.evamx_exl3_linear(FAKE, 65537, 2048, 7168, FAKE, FAKE, FAKE, 4.0, FAKE, FAKE, 1 << 40, None) == _lib.EVAMX_EINVAL
    assert L.evamx_exl3_linear(FAKE, 0, 2048, 7168, FAKE, FAKE, FAKE, 4.0, FAKE, FAKE, 1 << 30, None) == _lib.EVAMX_EINVAL
    assert L.evamx_exl3_linear(FAKE, 1, 2048, 7168, FAKE, FAKE, FAKE, 4.0, FAKE, FAKE, 16, None) == _lib.EVAMX_ENOSPACE
    assert L.evamx_route_topk(FAKE, 0, 1, 256, 300, 0, 1.0, FAKE, FAKE, FAKE, None) == _lib.EVAMX_EINVAL
    assert L.evamx_route_topk(FAKE, 0, 1, 600, 8, 0, 1.0, FAKE, FAKE, FAKE, None) == _lib.EVAMX_EINVAL
    assert L.evamx_prepare_routes(FAKE, FAKE, 5, 8, 4, 256, FAKE, FAKE, 1 << 20, None) == _lib.EVAMX_EINVAL
    assert L.evamx_prepare_routes(FAKE, FAKE, 4, 8, 4, 256, FAKE, FAKE, 8, None) == _lib.EVAMX_ENOSPACE
    assert L.evamx_moe_runs_ptr(ctypes.byref(_shape(hidden=1)), FAKE) is None
    assert L.evamx_moe_rotated_ptr(ctypes.byref(_shape(hidden=1)), FAKE) is None
    assert L.evamx_moe_rotated_ptr(ctypes.byref(_shape()), None) is None
    assert L.evamx_bench_decode(4.25, 4096, 10, FAKE, None) == _lib.EVAMX_EINVAL
    assert L.evamx_bench_decode(4.0, 4094, 10, FAKE, None) == _lib.EVAMX_EINVAL
    assert L.evamx_bench_decode(4.0, 4096, 0, FAKE, None) == _lib.EVAMX_EINVAL
    assert L.evamx_bench_decode(4.0, 4096, 10, None, None) == _lib.EVAMX_EINVAL
    assert L.evamx_bench_read(None, 1 << 20, 16, 4, 16, FAKE, None) == _lib.EVAMX_EINVAL
    assert L.evamx_bench_read(FAKE, 1 << 20, 16, 4, 24, FAKE, None) == _lib.EVAMX_EINVAL    # waves % ncg
    assert L.evamx_bench_read(FAKE, 1 << 20, 16, 0, 16, FAKE, None) == _lib.EVAMX_EINVAL    # rows
    assert L.evamx_bench_read(FAKE, (1 << 20) - 1, 16, 64, 16, FAKE, None) == _lib.EVAMX_EINVAL  # 1 MiB read
    assert L.evamx_router_logits(FAKE, _lib.DTYPE_BF16, 7168, 1, FAKE, 256, 7168, None, None) == _lib.EVAMX_EINVAL
    assert L.evamx_router_logits(FAKE, 5, 7168, 1, FAKE, 256, 7168, FAKE, None) == _lib.EVAMX_EINVAL
    assert L.evamx_router_logits(FAKE, _lib.DTYPE_BF16, 7168, 1, FAKE, 600, 7168, FAKE, None) == _lib.EVAMX_EINVAL
    assert L.evamx_router_logits(FAKE, _lib.DTYPE_BF16, 7100, 1, FAKE, 256, 7168, FAKE, None) == _lib.EVAMX_EINVAL
    assert L.evamx_router_logits(FAKE, _lib.DTYPE_BF16, 7168, 1, FAKE + 8, 256, 7168, FAKE, None) == _lib.EVAMX_EINVAL
    assert L.evamx_router_logits(FAKE, _lib.DTYPE_BF16, 7168, 0, FAKE, 256, 7168, FAKE, None) == _lib.EVAMX_EINVAL


def test_product_path_does_not_import_the_oracle():
    """The package never reaches the CPU restatement: no fallback exists to route through."""
    pkg = os.path.join(ROOT, "eva_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith(".py"):
                text = open(os.path.join(dirpath, f)).read()
                assert not re.search(r"^\s*(from|import)\s+oracle\b", text, flags=re.M), f


def test_runners_refuse_to_run_without_gpu():
    """No CPU numerical fallback: constructing a runner without a GPU raises."""
    import torch

    from eva_amd.coop import CoopRunner3072
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(RuntimeError, match="GPU"):
        CoopRunner3072("cuda:0", topk=6, hidden=256, inter=128, max_rows=4)
