"""Process-wide bound and switches for strict (batch-invariant) arithmetic.

Mirrors runtime/ds41/verification.py:15-30 (``DS41_VERIFY_MAX_ROWS``: the largest target input of
a speculative verification, read once at import; 1..128 or exactly 256/512/1024, default 8) and the
reference's strict switches: ``DS41_STRICT_BATCH`` (MoE, default on: moe_coop.py:17-22,
cache.py:2088-2091) and ``DS41_STRICT_DENSE`` (EXL3 linears, default on: exl3_linear.py:70).

In strict mode a row's result does not depend on how many rows share its call, up to the bound:
the MoE runs every such call through the arithmetic of a one-row call (``strict_rows`` of the
workspace), and ``ELinear`` keeps such calls on the decode GEMV, whose per-row arithmetic depends
on in/out only.
"""
from __future__ import annotations

import os

MAX_VERIFICATION_ROWS = 1024
LEGACY_MAX_VERIFICATION_ROWS = 128
# Strict MoE calls run on the decode path's one-workgroup prepare: EVAMX_STRICT_MAX_ROWS and
# EVAMX_STRICT_MAX_SLOTS of include/evamx.h.
STRICT_MOE_MAX_ROWS = 64
STRICT_MOE_MAX_SLOTS = 256

_MSG = "DS41_VERIFY_MAX_ROWS must be an integer from 1 to 128 or explicit 256/512/1024"


def parse_max_rows(value) -> int:
    """The reference's accepted values: the integer's own spelling, 1..128, or 256, 512, 1024."""
    if not isinstance(value, str):
        raise ValueError(_MSG)
    try:
        rows = int(value)
    except (TypeError, ValueError) as exc:
        raise ValueError(_MSG) from exc
    if str(rows) != value.strip() or not (1 <= rows <= LEGACY_MAX_VERIFICATION_ROWS or rows in (256, 512, 1024)):
        raise ValueError(_MSG)
    return rows


_MAX_ROWS = parse_max_rows(os.environ.get("DS41_VERIFY_MAX_ROWS", "8"))


def verification_max_rows() -> int:
    """The startup-validated verification row bound (pending + proposals)."""
    return _MAX_ROWS


def strict_batch() -> bool:
    """DS41_STRICT_BATCH (default "1"): MoE rows bit-identical across batch sizes up to the bound."""
    return os.environ.get("DS41_STRICT_BATCH", "1") == "1"


def strict_dense() -> bool:
    """DS41_STRICT_DENSE (default on, "0" turns it off): EXL3 linear rows likewise."""
    return os.environ.get("DS41_STRICT_DENSE", "1") != "0"


def moe_strict_rows(max_rows: int, topk: int, strict: bool | None = None, bound: int | None = None) -> int:
    """The ``strict_rows`` of a MoE workspace of ``max_rows`` rows at ``topk``: 0 when strict mode
    is off, else min(max_rows, bound). A bound beyond what strict mode covers is an error, never
    silently narrowed (the reference refuses an explicitly different target, cache.py:2088-2091)."""
    strict = strict_batch() if strict is None else strict
    if not strict:
        return 0
    rows = min(max_rows, verification_max_rows() if bound is None else bound)
    if rows > STRICT_MOE_MAX_ROWS or rows * topk > STRICT_MOE_MAX_SLOTS:
        raise ValueError(f"strict MoE batches cover at most {STRICT_MOE_MAX_ROWS} rows and {STRICT_MOE_MAX_SLOTS} "
                         f"slots; {rows} rows at top-{topk} need more: lower DS41_VERIFY_MAX_ROWS or set "
                         "DS41_STRICT_BATCH=0")
    return rows
