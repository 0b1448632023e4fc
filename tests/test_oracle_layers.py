"""Routing, expert FFN and MoE-layer parts of the oracle (no GPU).

Pinned by the reference's operator fixture (tests/golden/deepseek_v4_moe_operators.json, copied
from the reference's tests/fixtures/deepseek_v4_operators.json), by closed forms, and by an
independent float64 numpy restatement of the combine loops, built on decoded weights.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest

from oracle.oracle import (F32, IQ1_S, IQ2_XXS, IQ3_XXS, Q8_0, SCORE_SIGMOID,
                           SCORE_SQRT_SOFTPLUS, OracleError)
from vastloom_amd.workloads import random_matrix

GOLDEN = json.loads((Path(__file__).parent / "golden" / "deepseek_v4_moe_operators.json").read_text())
ATOL = GOLDEN["absolute_tolerance"]


def f32_matrix(values) -> tuple[int, np.ndarray]:
    return F32, np.ascontiguousarray(values, np.float32).view(np.uint8)


def test_fixture_clamped_swiglu_expert(oracle):
    e = GOLDEN["expert"]
    H, F, T = e["width"], e["intermediate"], e["tokens"]
    y = oracle.expert_deepseek(f32_matrix(e["gate_weight"]), f32_matrix(e["up_weight"]),
                               f32_matrix(e["down_weight"]), H, F,
                               np.array(e["input"], np.float32).reshape(T, H),
                               routing=e["routing_weights"], limit=e["swiglu_limit"])
    assert np.allclose(y.reshape(-1), e["expected"], atol=ATOL, rtol=0)


def test_fixture_hash_route(oracle):
    r = GOLDEN["hash_route"]
    logits = oracle.linear_f64(r["gate_weight"], np.array(r["input"], np.float32), r["experts"])
    idx, w = oracle.route_hash(logits, r["token_ids"], r["token_to_experts"], r["top_k"],
                               r["route_scale"], SCORE_SQRT_SOFTPLUS)
    assert idx.reshape(-1).tolist() == r["expected_indices"]
    assert np.allclose(w.reshape(-1), r["expected_weights"], atol=ATOL, rtol=0)


def test_fixture_learned_route(oracle):
    r = GOLDEN["learned_route"]
    logits = oracle.linear_f64(r["gate_weight"], np.array(r["input"], np.float32), r["experts"])
    idx, w = oracle.route_learned(logits, r["selection_bias"], r["top_k"], r["route_scale"],
                                  SCORE_SQRT_SOFTPLUS)
    assert idx.reshape(-1).tolist() == r["expected_indices"]
    assert np.allclose(w.reshape(-1), r["expected_weights"], atol=ATOL, rtol=0)


@pytest.mark.parametrize("v", [-30.0, -5.5, -1e-3, 0.0, 1e-3, 0.7, 4.0, 30.0])
def test_scoring_closed_forms(oracle, v):
    sp = math.sqrt(max(v, 0.0) + math.log1p(math.exp(-abs(v))))
    assert oracle.sqrt_softplus(v) == np.float32(sp)
    sg = 1.0 / (1.0 + math.exp(-v)) if v >= 0 else math.exp(v) / (1.0 + math.exp(v))
    assert oracle.sigmoid(v) == np.float32(sg)
    # silu_f is float arithmetic; compare to float64 within a few ulps.
    ref = v / (1.0 + math.exp(-v))
    assert abs(oracle.silu_f(v) - ref) <= 4 * np.spacing(np.float32(abs(ref)) + np.float32(1e-30))


def test_route_invariants(oracle):
    rng = np.random.default_rng(7)
    logits = rng.standard_normal((6, 32)).astype(np.float32)
    bias = (rng.standard_normal(32) * 0.1).astype(np.float32)
    for fn in (SCORE_SQRT_SOFTPLUS, SCORE_SIGMOID):
        idx, w = oracle.route_learned(logits, bias, 4, 2.5, fn)
        act = (np.vectorize(oracle.sigmoid if fn else oracle.sqrt_softplus)(logits)
               ).astype(np.float32)
        for t in range(6):
            key = act[t] + bias
            # Brute force: the four largest keys, ties to the lower id.
            order = sorted(range(32), key=lambda e: (-key[e], e))[:4]
            assert idx[t].tolist() == order
            sel = act[t, order].astype(np.float64)
            assert np.allclose(w[t], (sel / sel.sum() * 2.5).astype(np.float32), rtol=0, atol=0)
    # Ties go to the lower id.
    tie = np.zeros((1, 8), np.float32)
    idx, w = oracle.route_learned(tie, None, 3, 1.0, SCORE_SIGMOID)
    assert idx[0].tolist() == [0, 1, 2]
    assert np.allclose(w, 1 / 3)
    with pytest.raises(OracleError):
        oracle.route_learned(tie, None, 9, 1.0, SCORE_SIGMOID)
    bad = tie.copy()
    bad[0, 3] = np.inf
    with pytest.raises(OracleError):
        oracle.route_learned(bad, None, 2, 1.0, SCORE_SIGMOID)


def test_route_softmax_matches_float64(oracle):
    rng = np.random.default_rng(11)
    logits = (rng.standard_normal(64) * 2).astype(np.float32)
    idx, w = oracle.route_softmax(logits, 8, True)
    p = np.exp(logits.astype(np.float64) - logits.max())
    p /= p.sum()
    order = sorted(range(64), key=lambda e: (-p[e], e))[:8]
    assert idx.tolist() == order
    top = p[order]
    assert np.allclose(w, top.astype(np.float32).astype(np.float64) / top.sum(), rtol=1e-7)


def _decoded(oracle, qtype, data, rows, cols):
    return oracle.dequantize(qtype, data, rows * cols).reshape(rows, cols).astype(np.float64)


def _np_expert_deepseek(oracle, w, H, F, x, route, limit):
    """Float64 restatement of execute_expert on decoded weights."""
    (t1, b1), (t3, b3), (t2, b2) = w
    g = (_decoded(oracle, t1, b1, F, H) @ x.astype(np.float64)).astype(np.float32)
    u = (_decoded(oracle, t3, b3, F, H) @ x.astype(np.float64)).astype(np.float32)
    gv, uv = g.astype(np.float64), u.astype(np.float64)
    if limit > 0:
        gv = np.minimum(gv, limit)
        uv = np.clip(uv, -limit, limit)
    h = gv / (1.0 + np.exp(-gv)) * uv
    if route is not None:
        h = h * np.float64(np.float32(route))
    h = h.astype(np.float32)
    return (_decoded(oracle, t2, b2, H, F) @ h.astype(np.float64)).astype(np.float32)


@pytest.mark.parametrize("qtypes", [(IQ2_XXS, IQ2_XXS), (IQ1_S, IQ3_XXS), (Q8_0, Q8_0)])
def test_moe_deepseek_against_numpy(oracle, qtypes):
    rng = np.random.default_rng(5)
    H, F, E, K, T = 512, 256, 6, 2, 3
    gt, dt = qtypes
    experts = [((gt, random_matrix(rng, gt, F, H, 0.01)), (gt, random_matrix(rng, gt, F, H, 0.01)),
                (dt, random_matrix(rng, dt, H, F, 0.01))) for _ in range(E)]
    shared = experts[0]
    x = rng.standard_normal((T, H)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    idx, w = oracle.route_learned(logits, None, K, 1.0, SCORE_SIGMOID)
    out = oracle.moe_deepseek(x, idx, w, experts, shared, H, F, routed_limit=0.0)
    for t in range(T):
        want = np.zeros(H, np.float32)
        for e in range(E):
            for s in range(K):
                if idx[t, s] == e:
                    want += _np_expert_deepseek(oracle, experts[e], H, F, x[t], w[t, s], 0.0)
        want += _np_expert_deepseek(oracle, shared, H, F, x[t], None, 0.0)
        scale = np.abs(want).max()
        assert np.allclose(out[t], want, atol=1e-5 * scale, rtol=0)


def test_moe_qwen_against_numpy(oracle):
    rng = np.random.default_rng(9)
    H, F, E, K = 256, 128, 8, 3
    experts = [tuple((Q8_0, random_matrix(rng, Q8_0, r, c, 0.002))
                     for r, c in ((F, H), (F, H), (H, F))) for _ in range(E)]
    x = rng.standard_normal(H).astype(np.float32)
    logits = rng.standard_normal(E).astype(np.float32)
    idx, w = oracle.route_softmax(logits, K, True)
    out = oracle.moe_qwen(x, idx, w, experts, None, H, F)
    want = np.zeros(H, np.float32)
    for s in range(K):
        (tg, bg), (tu, bu), (td, bd) = experts[idx[s]]
        g = (_decoded(oracle, tg, bg, F, H) @ x.astype(np.float64)).astype(np.float32)
        u = (_decoded(oracle, tu, bu, F, H) @ x.astype(np.float64)).astype(np.float32)
        h = (np.vectorize(oracle.silu_f)(g).astype(np.float32) * u).astype(np.float32)
        y = (_decoded(oracle, td, bd, H, F) @ h.astype(np.float64)).astype(np.float32)
        want = (want + (y * w[s]).astype(np.float32)).astype(np.float32)
    assert np.allclose(out, want, atol=1e-6 * np.abs(want).max(), rtol=0)


def test_moe_rejects_out_of_range_expert(oracle):
    rng = np.random.default_rng(1)
    H, F = 256, 256
    e = tuple((IQ2_XXS, random_matrix(rng, IQ2_XXS, r, c, 0.01)) for r, c in ((F, H), (F, H), (H, F)))
    with pytest.raises(OracleError):
        oracle.moe_deepseek(np.ones((1, H), np.float32), np.array([[3]]), np.array([[1.0]]),
                            [e], None, H, F)
