"""Brute-force restatement of the reference forward in pure Python floats.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`).

Nested loops over Python lists with `math.exp`, `math.erf` and `math.sqrt` in
double precision. It shares no code with `oracle.reference` and uses no torch
arithmetic, so agreement between the two pins `reference` against a plain
reading of `torch_transformer_benchmark.py:85-172`. Only for tiny shapes
(B <= 2, S <= 8, d <= 16): the cost is O(L * B * S^2 * d + L * B * S * d * F).
"""
from __future__ import annotations

import math
from typing import Dict, List, Optional

Mat = List[List[float]]


def _lin(x: List[float], w: Mat, b: List[float]) -> List[float]:
    return [sum(x[k] * w[n][k] for k in range(len(x))) + b[n] for n in range(len(w))]


def _ln(x: List[float], g: List[float], b: List[float], eps: float) -> List[float]:
    n = len(x)
    mean = sum(x) / n
    var = sum((v - mean) ** 2 for v in x) / n
    r = 1.0 / math.sqrt(var + eps)
    return [(x[i] - mean) * r * g[i] + b[i] for i in range(n)]


def _gelu(v: float) -> float:
    return 0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0)))


def forward(p: Dict[str, list], x: List[List[List[float]]],
            mask: Optional[List[List[bool]]], num_heads: int, causal: bool,
            eps: float = 1e-5) -> List[List[List[float]]]:
    """x: [B][S][d] nested lists; p: state-dict names -> nested lists."""
    B, S, d = len(x), len(x[0]), len(x[0][0])
    H = num_heads
    Dh = d // H
    L = 0
    while f"layers.{L}.norm1.weight" in p:
        L += 1
    valid = [[True] * S for _ in range(B)] if mask is None else mask
    x = [[list(row) for row in seq] for seq in x]
    for i in range(L):
        pre = f"layers.{i}."
        g = lambda name: p[pre + name]  # noqa: E731
        for bi in range(B):
            n1 = [_ln(x[bi][s], g("norm1.weight"), g("norm1.bias"), eps) for s in range(S)]
            q = [_lin(n1[s], g("attention.q_proj.weight"), g("attention.q_proj.bias")) for s in range(S)]
            k = [_lin(n1[s], g("attention.k_proj.weight"), g("attention.k_proj.bias")) for s in range(S)]
            v = [_lin(n1[s], g("attention.v_proj.weight"), g("attention.v_proj.bias")) for s in range(S)]
            ctx = [[0.0] * d for _ in range(S)]
            for h in range(H):
                lo = h * Dh
                for s in range(S):
                    scores = []
                    for t in range(S):
                        ok = valid[bi][t] and (not causal or t <= s)
                        if ok:
                            dot = sum(q[s][lo + j] * k[t][lo + j] for j in range(Dh))
                            scores.append(dot / math.sqrt(Dh))
                        else:
                            scores.append(None)
                    live = [z for z in scores if z is not None]
                    if not live:          # every key masked: the reference gives NaN
                        for j in range(Dh):
                            ctx[s][lo + j] = float("nan")
                        continue
                    m = max(live)
                    e = [0.0 if z is None else math.exp(z - m) for z in scores]
                    tot = sum(e)
                    for j in range(Dh):
                        ctx[s][lo + j] = sum(e[t] / tot * v[t][lo + j] for t in range(S))
            attn = [_lin(ctx[s], g("attention.out_proj.weight"), g("attention.out_proj.bias")) for s in range(S)]
            for s in range(S):
                if not valid[bi][s]:
                    attn[s] = [0.0] * d
                x[bi][s] = [x[bi][s][j] + attn[s][j] for j in range(d)]
            for s in range(S):
                n2 = _ln(x[bi][s], g("norm2.weight"), g("norm2.bias"), eps)
                hid = [_gelu(z) for z in _lin(n2, g("ffn_in.weight"), g("ffn_in.bias"))]
                f = _lin(hid, g("ffn_out.weight"), g("ffn_out.bias"))
                x[bi][s] = [x[bi][s][j] + f[j] for j in range(d)]
                if not valid[bi][s]:
                    x[bi][s] = [0.0] * d
    out = []
    for bi in range(B):
        rows = []
        for s in range(S):
            r = _ln(x[bi][s], p["final_norm.weight"], p["final_norm.bias"], eps)
            rows.append(r if valid[bi][s] else [0.0] * d)
        out.append(rows)
    return out
