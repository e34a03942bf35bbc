"""All-resident expert store with the reference ExpertCache's MoE entry point.

Replaces ``ExpertCache`` (runtime/ds41/cache.py:107-2382) on the path this build covers:
``moe(layer, x, indices, weights, k, limit, inter)`` (cache.py:2276) returns the routed
experts' fp32 sum ``[rows, hidden]`` from the ``[L, 9, N]`` pointer tables ``packed``
(cache.py:237-238, rows g/u/d x trellis/suh/svh as bound at cache.py:1864-1886).

The reference pages experts between NVMe, pinned RAM and a VRAM cache and binds a layer's
pointers before each call. A 288 GB MI355X holds every expert of the model, so this store
loads the requested layers of a DS41PK01 pack into HBM once (``eva_amd.pack.load_layers``) and
the pointer tables never change: there is no ``_flush`` before a call, no routes readback
(cache.py:2315's ``indices.tolist()``) and no host synchronisation, so ``moe`` and ``moe_step``
can be captured into a hipGraph. Rates come from the pack per expert (mixed-rate packs work);
``k``, when given, must match them.

``moe_step`` is the fused form a decode step uses: routing on the device from gate logits or
from the router weight itself (``Block.route``, model.py:404-416), the routed experts, and
optionally the shared expert (``Block._shared``, model.py:418-452, added at model.py:498).
"""
from __future__ import annotations

import torch

from . import ops, verification
from .pack import PackIndex, load_layers, read_index


class ResidentExperts:
    """Experts of ``layers`` of a DS41PK01 pack (default all) resident on ``device``."""

    def __init__(self, pack, device=None, layers=None, topk: int = 8, max_rows: int = 16, *,
                 strict_rows: int | None = None):
        """``strict_rows`` None follows DS41_STRICT_BATCH / DS41_VERIFY_MAX_ROWS (calls of up to the
        verification bound give every row a one-row call's bits); 0 turns strict mode off."""
        index = pack if isinstance(pack, PackIndex) else read_index(pack)
        self.index = index
        self.device = torch.device("cuda", 0) if device is None else torch.device(device)
        self.layer_ids = list(range(index.n_layers) if layers is None else layers)
        self._layers = dict(zip(self.layer_ids, load_layers(index, self.layer_ids, self.device)))
        first = self._layers[self.layer_ids[0]]
        self.hidden, self.inter = first.hidden, first.inter
        self.n_experts = index.n_experts
        self.topk = topk
        self.max_rows = max_rows
        self.strict_rows = strict_rows
        # [L, 9, N] pointer tables and [L, N] rates (2 x bits) of the resident layers, in layer order
        self.packed = torch.stack([self._layers[l].table for l in self.layer_ids])
        self.k2 = torch.stack([self._layers[l].k2 for l in self.layer_ids])
        self.k2_down = torch.stack([self._layers[l].k2_down for l in self.layer_ids])
        self._pos = {l: i for i, l in enumerate(self.layer_ids)}
        self._rates = {l: set(self._layers[l].k2_host) for l in self.layer_ids}
        self._ws = {}

    def _workspace(self, rows: int, topk: int, has_shared: bool):
        key = (topk, has_shared)
        ws = self._ws.get(key)
        if ws is None or ws.shape.rows_max < rows:
            cap = max(rows, self.max_rows)
            strict = (verification.moe_strict_rows(cap, topk) if self.strict_rows is None
                      else min(self.strict_rows, cap))
            ws = ops.MoeWorkspace(self.device, rows_max=cap, hidden=self.hidden, inter=self.inter, topk=topk,
                                  n_local=self.n_experts, has_shared=has_shared, strict_rows=strict)
            self._ws[key] = ws
        return ws

    def _layer(self, layer: int):
        if layer not in self._pos:
            raise KeyError(f"layer {layer} is not resident (loaded: {self.layer_ids})")
        i = self._pos[layer]
        return self.packed[i], self.k2[i], self.k2_down[i]

    def _check(self, x, k, inter):
        if inter is not None and inter != self.inter:
            raise ValueError(f"inter {inter} does not match the pack ({self.inter})")
        if x.shape[-1] != self.hidden:
            raise ValueError(f"x has {x.shape[-1]} features, the pack {self.hidden}")

    def _check_rate(self, layer, k):
        if k is None:
            return
        want = int(round(2 * float(k)))
        if self._rates[layer] != {want}:
            raise ValueError(f"k={k} does not match layer {layer}'s rates "
                             f"{sorted(r / 2 for r in self._rates[layer])}")

    def moe(self, layer, x, indices, weights, k=None, limit=0.0, inter=None, *, out=None) -> torch.Tensor:
        """Routed experts of ``layer`` for given routes: fp32 ``[rows, hidden]`` (cache.py:2276).
        ``indices`` int ``[..., topk]`` (local expert ids), ``weights`` float ``[..., topk]``."""
        self._check(x, k, inter)
        table, k2, k2d = self._layer(layer)
        self._check_rate(layer, k)
        x2 = x.reshape(-1, self.hidden)
        if x2.dtype not in (torch.float16, torch.bfloat16):
            x2 = x2.to(torch.float16)
        rows = x2.shape[0]
        topk = indices.shape[-1]
        sel = indices.reshape(rows, topk).to(device=self.device, dtype=torch.int64).contiguous()
        w = weights.reshape(rows, topk).to(device=self.device, dtype=torch.float32).contiguous()
        ws = self._workspace(rows, topk, False)
        if out is None:
            out = torch.empty(rows, self.hidden, dtype=torch.float32, device=self.device)
        ops.moe_forward(ws, x2.contiguous(), table, out, limit=float(limit), k2_per_expert=k2, k2_down_per_expert=k2d,
                        sel=sel, weights=w)
        return out

    def moe_step(self, layer, x, logits=None, *, gate_w=None, limit=0.0, score_fn="sigmoid", sel_bias=None,
                 route_scale=1.0, shared=None, shared_bits=None, residual=None, out=None, sel=None, weights=None):
        """Route on the device from fp32 ``logits [rows, n_experts]``, or from the router weight
        ``gate_w`` (fp32 ``[n_experts, hidden]``: the logits ``x.float() @ gate_w.T`` are computed
        in the same call, model.py:404-409), and run the routed experts plus, when ``shared``
        (9 device pointers) is given, the shared expert. With ``residual`` (bf16 ``[rows, hidden]``,
        may be ``x``) the output is added into it in place. Returns ``(out, sel, weights)``;
        capturable into a hipGraph (no host synchronisation)."""
        self._check(x, None, None)
        table, k2, k2d = self._layer(layer)
        rows = x.shape[0]
        ws = self._workspace(rows, self.topk, shared is not None)
        if sel is None:
            sel = torch.empty(rows, self.topk, dtype=torch.int64, device=self.device)
        if weights is None:
            weights = torch.empty(rows, self.topk, dtype=torch.float32, device=self.device)
        if out is None and residual is None:
            out = torch.empty(rows, self.hidden, dtype=torch.float32, device=self.device)
        if (logits is None) == (gate_w is None):
            raise ValueError("give logits or gate_w")
        ops.moe_forward(ws, x, table, out, limit=float(limit), k2_per_expert=k2, k2_down_per_expert=k2d,
                        logits=logits, gate_w=gate_w,
                        sel=sel, weights=weights, score_fn=score_fn, sel_bias=sel_bias, route_scale=route_scale,
                        shared_ptrs=shared, shared_bits=shared_bits, residual=residual)
        return out, sel, weights

    def flags(self, topk=None, has_shared=False) -> int:
        """Sticky device error flags of the workspace (EVAMX_ERR_*); reads the device."""
        ws = self._ws.get((self.topk if topk is None else topk, has_shared))
        return 0 if ws is None else int(ws.flags().cpu()[0])
