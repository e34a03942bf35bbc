"""Seeded synthetic inputs for the benchmark configurations (test infrastructure; numpy).

The GPU tests generate inputs here, upload them, and compare against the oracle on the
same arrays. ``bench.py`` generates its (much larger) inputs on the device with the same
distributions; parity at those sizes is checked through size-independent properties.

Distributions of the benchmark configurations:

- trellis: uniform int16 over all 65 536 values, ``[in/16, out/16, T]``;
- suh: Rademacher +-1 (fp16); svh: +-1 * U(0.5, 1.5) * svh_scale (fp16);
- activations: bf16 ~ N(0, 1); router logits fp32 ~ N(0, 1).
"""
from __future__ import annotations

import numpy as np

from . import exl3
from .coop import ExpertWeights


def projection(rng, n_in, n_out, K, svh_scale=1.0):
    t16 = exl3.tile_u16(K)
    trellis = rng.integers(-32768, 32768, size=(n_in // 16, n_out // 16, t16), dtype=np.int16)
    suh = rng.choice(np.array([-1.0, 1.0]), size=n_in).astype(np.float16)
    mag = rng.uniform(0.5, 1.5, size=n_out) * svh_scale
    svh = (rng.choice(np.array([-1.0, 1.0]), size=n_out) * mag).astype(np.float16)
    return trellis, suh, svh


def expert(rng, hidden, inter, K, svh_scale=1.0, K_down=None):
    """Gate and up at rate K, down at K_down (default K)."""
    Kd = K if K_down is None else K_down
    g = projection(rng, hidden, inter, K, svh_scale)
    u = projection(rng, hidden, inter, K, svh_scale)
    d = projection(rng, inter, hidden, Kd, svh_scale)
    return ExpertWeights(g, u, d, K, Kd)


def activations_bf16(rng, t, hidden):
    """bf16 ~ N(0,1), returned as float32 values exactly representable in bf16 (RNE)."""
    x = rng.standard_normal((t, hidden)).astype(np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def logits_plain(rng, t, n_experts):
    return rng.standard_normal((t, n_experts)).astype(np.float32)


def logits_skewed(rng, t, n_experts, hot=2, warm=6):
    """Config 3: a per-token random bias on top of N(0,1) so that expert loads span 0..T.

    ``hot`` experts get +6 (every token picks them), ``warm`` experts get a per-token
    Bernoulli(1/2) bias of +3 (about half the tokens pick each), the rest only noise.
    """
    z = rng.standard_normal((t, n_experts)).astype(np.float32)
    perm = rng.permutation(n_experts)
    z[:, perm[:hot]] += 6.0
    coin = rng.integers(0, 2, size=(t, warm)).astype(np.float32)
    z[:, perm[hot:hot + warm]] += 3.0 * coin
    return z


def logits_zipf(rng, t, n_experts, s=1.1):
    """Config 4: Zipf(s) over a random expert permutation, k distinct picks per token.

    ``log p_e + Gumbel`` noise: the top-k of these logits is a draw of k distinct experts
    without replacement with probabilities proportional to p (the Gumbel-top-k identity).
    """
    ranks = np.arange(1, n_experts + 1, dtype=np.float64)
    p = ranks ** (-s)
    p /= p.sum()
    perm = rng.permutation(n_experts)
    logp = np.empty(n_experts)
    logp[perm] = np.log(p)
    g = rng.gumbel(size=(t, n_experts))
    return (logp[None, :] + g).astype(np.float32)


def mixed_rates(rng, n_experts, rates=(2, 3, 4, 5)):
    """Per-expert rates drawn uniformly from ``rates`` (config 4: {2,3,4,5})."""
    return rng.choice(np.array(rates, dtype=np.float64), size=n_experts)
