"""Helpers shared by the MoE parity tests: oracle layer outputs with their tolerance bounds, and
device layers built from the same bytes."""

from __future__ import annotations

import numpy as np

from oracle.oracle import SCORE_SIGMOID, SCORE_SQRT_SOFTPLUS

TOL = 1e-5


def silu_f_vec(oracle, g: np.ndarray) -> np.ndarray:
    return np.array([oracle.silu_f(float(v)) for v in g], np.float32)


def expert_h(oracle, sem: str, triple, width, inter, x, route_w=None, limit=0.0):
    """The oracle's intermediate activation of one expert for one token (float32)."""
    (tg, g_bytes), (tu, u_bytes), _ = triple
    g = oracle.matvec(tg, g_bytes, inter, width, x, threads=8)
    u = oracle.matvec(tu, u_bytes, inter, width, x, threads=8)
    if sem == "deepseek":
        gv, uv = g.astype(np.float64), u.astype(np.float64)
        if limit > 0:
            gv = np.minimum(gv, limit)
            uv = np.clip(uv, -limit, limit)
        h = gv / (1.0 + np.exp(-gv)) * uv
        if route_w is not None:
            h = h * np.float64(np.float32(route_w))
        return h.astype(np.float32)
    if sem == "qwen":
        return (silu_f_vec(oracle, g) * u).astype(np.float32)
    return (g / (np.float32(1.0) + np.exp(-g)) * u).astype(np.float32)


def down_row_norms(oracle, triple, width, inter) -> np.ndarray:
    td, d_bytes = triple[2]
    w = oracle.dequantize(td, d_bytes, width * inter).reshape(width, inter)
    return np.linalg.norm(w.astype(np.float64), axis=1)


def layer_bound(oracle, sem, experts, shared, ids, weights, x, width, inter,
                routed_limit=0.0, shared_limit=0.0) -> np.ndarray:
    """Per-element bound TOL * sum over contributing experts of |down_row| * |h|, the row
    tolerance of each down projection carried through the combine."""
    tokens = x.shape[0]
    bound = np.zeros((tokens, width))
    norms = {}
    for t in range(tokens):
        for s in range(ids.shape[1]):
            e = int(ids[t, s])
            rw = weights[t, s] if sem == "deepseek" else None
            h = expert_h(oracle, sem, experts[e], width, inter, x[t], rw, routed_limit)
            if e not in norms:
                norms[e] = down_row_norms(oracle, experts[e], width, inter)
            scale = abs(float(weights[t, s])) if sem == "qwen" else 1.0
            bound[t] += TOL * norms[e] * np.linalg.norm(h.astype(np.float64)) * scale
        if shared is not None:
            h = expert_h(oracle, sem, shared, width, inter, x[t], None, shared_limit)
            if "shared" not in norms:
                norms["shared"] = down_row_norms(oracle, shared, width, inter)
            bound[t] += TOL * norms["shared"] * np.linalg.norm(h.astype(np.float64))
    return bound


def oracle_routes(oracle, routing, logits, top_k, score_fn, bias=None, table=None,
                  route_scale=1.0, renormalize=True):
    if routing == "softmax":
        ids, w = zip(*(oracle.route_softmax(l, top_k, renormalize) for l in logits))
        return np.stack(ids), np.stack(w)
    if routing == "table":
        return oracle.route_hash(logits, np.arange(len(table)), table, top_k, route_scale,
                                 score_fn)
    return oracle.route_learned(logits, bias, top_k, route_scale, score_fn)


SCORES = {"sigmoid": SCORE_SIGMOID, "sqrt_softplus": SCORE_SQRT_SOFTPLUS}
