"""Expert FFNs and MoE layers on the MI355X against the oracle, through the C ABI.

Routing must select the same experts as the oracle with weights equal to float rounding; layer
outputs must stay within the tolerance the path is specified with (1e-5 * |w_row| * |x| for each
down projection, carried through the combine). Full-size cases are the benchmark workloads:
OLMoE-shaped Q8_0 expert and 64-expert layer, DeepSeek-shaped IQ2_XXS and IQ1_S/IQ3_XXS layers.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.oracle import (BF16, IQ1_S, IQ2_S, IQ2_XXS, IQ3_XXS, MXFP4, Q4_K, Q5_K, Q6_K, Q8_0,
                           SCORE_SIGMOID, SCORE_SQRT_SOFTPLUS)
from tests.moe_cases import TOL, down_row_norms, expert_h, layer_bound, oracle_routes
from vastloom_amd.workloads import random_matrix, workload

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    assert torch.cuda.is_available(), "GPU tests need a visible HIP device"
    from vastloom_amd import ops as _ops

    return _ops


@pytest.fixture(scope="module")
def lib():
    from vastloom_amd import _lib

    return _lib


def make_expert(rng, gt, dt, H, F, scale=0.01):
    return ((gt, random_matrix(rng, gt, F, H, scale)), (gt, random_matrix(rng, gt, F, H, scale)),
            (dt, random_matrix(rng, dt, H, F, scale)))


def device_expert(ops, triple, H, F):
    (gt, g), (_, u), (dt, d) = triple
    return ops.DeviceExpert(gt, dt, H, F, g, u, d)


SEMS = {"deepseek": 0, "qwen": 1, "plain": 2}


@pytest.mark.parametrize("gt,dt", [(IQ2_XXS, IQ2_XXS), (IQ1_S, IQ3_XXS), (IQ1_S, IQ1_S), (Q8_0, Q8_0),
                                   # GGUF-layout types, alone and under tiled gate/up matrices
                                   (Q4_K, Q6_K), (Q5_K, Q4_K), (IQ2_S, IQ2_S), (BF16, MXFP4),
                                   (IQ2_XXS, MXFP4), (IQ1_S, Q6_K)])
@pytest.mark.parametrize("sem", ["deepseek", "qwen", "plain"])
@pytest.mark.parametrize("tokens", [1, 3])
def test_expert_ffn(ops, lib, oracle, gt, dt, sem, tokens):
    print(f"[expert_ffn] {gt}/{dt} {sem} tokens={tokens}", flush=True)
    rng = np.random.default_rng(gt * 100 + dt + tokens)
    H, F = 1024, 512
    triple = make_expert(rng, gt, dt, H, F)
    x = rng.standard_normal((tokens, H)).astype(np.float32)
    route = (rng.random(tokens) + 0.25).astype(np.float32)
    limit = 0.0
    if sem == "deepseek":
        limit = 0.05
        want = oracle.expert_deepseek(*triple, H, F, x, routing=route, limit=limit)
    elif sem == "qwen":
        want = np.stack([oracle.expert_qwen(*triple, H, F, x[t]) for t in range(tokens)])
    else:
        want = np.stack([oracle.routed_expert_iq1s_iq3xxs(triple[0][1], triple[1][1], triple[2][1],
                                                          H, F, x[t])
                         if (gt, dt) == (IQ1_S, IQ3_XXS) else
                         _plain_ffn(oracle, triple, H, F, x[t]) for t in range(tokens)])
    dev = device_expert(ops, triple, H, F)
    rw = torch.from_numpy(route).cuda() if sem == "deepseek" else None
    got = ops.expert_ffn(dev, torch.from_numpy(x).cuda(), semantics=SEMS[sem],
                         route_weights=rw, limit=limit).cpu().numpy()
    norms = down_row_norms(oracle, triple, H, F)
    for t in range(tokens):
        h = expert_h(oracle, sem, triple, H, F, x[t], route[t] if sem == "deepseek" else None, limit)
        bound = TOL * norms * np.linalg.norm(h.astype(np.float64))
        err = np.abs(got[t].astype(np.float64) - want[t])
        assert np.all(err <= bound), float((err / bound).max())


def _plain_ffn(oracle, triple, H, F, x):
    h = expert_h(oracle, "plain", triple, H, F, x)
    (td, d) = triple[2]
    return oracle.matvec(td, d, H, F, h)


def _device_layer(ops, lib, wl, experts, shared, sem, routing, router=None, bias=None,
                  score_fn=SCORE_SIGMOID, route_scale=1.0, routed_limit=0.0, shared_limit=0.0):
    H, F = wl.width, wl.intermediate
    devs = [device_expert(ops, e, H, F) for e in experts]
    sh = device_expert(ops, shared, H, F) if shared is not None else None
    torch.cuda.synchronize()
    for d in devs + ([sh] if sh else []):
        d.release_staging()
    return ops.MoeLayer(devs, sh, width=H, intermediate=F, top_k=wl.top_k,
                        gate_type=wl.gate_type, down_type=wl.down_type, semantics=SEMS[sem],
                        routing=routing, score_fn=score_fn, route_scale=route_scale,
                        routed_limit=routed_limit, shared_limit=shared_limit,
                        router=None if router is None else torch.from_numpy(router),
                        bias=None if bias is None else torch.from_numpy(bias))


def _check_layer(ops, lib, oracle, wl, experts, shared, sem, routing_name, routing, x,
                 score_fn=SCORE_SIGMOID, bias=None, table=None, route_scale=1.0,
                 routed_limit=0.0, shared_limit=0.0, sample=None, router=None):
    """Routes of every token must equal the oracle's; outputs are checked for every token, or
    for the tokens in `sample` (each token's output depends on its own routes only)."""
    H, F = wl.width, wl.intermediate
    router = wl.router() if router is None else router
    layer = _device_layer(ops, lib, wl, experts, shared, sem, routing, router, bias, score_fn,
                          route_scale, routed_limit, shared_limit)
    xt = torch.from_numpy(x).cuda()
    tab = None if table is None else torch.from_numpy(np.ascontiguousarray(table, np.uint32)).cuda()
    got = layer.forward(xt, table_ids=tab).cpu().numpy()
    ids_dev, w_dev = layer.routes(x.shape[0])
    logits = oracle.linear_f64(router, x, wl.experts)
    ids, w = oracle_routes(oracle, routing_name, logits, wl.top_k, score_fn, bias, table,
                           route_scale)
    assert np.array_equal(ids_dev, ids), (ids_dev, ids)
    assert np.allclose(w_dev, w, rtol=1e-6, atol=0)
    if sample is not None:
        sample = np.asarray(sample)
        got, x, ids, w = got[sample], x[sample], ids[sample], w[sample]
    if sem == "qwen":
        want = np.stack([oracle.moe_qwen(x[t], ids[t], w[t], experts, shared, H, F, threads=8)
                         for t in range(x.shape[0])])
    else:
        want = oracle.moe_deepseek(x, ids, w, experts, shared, H, F, routed_limit=routed_limit,
                                   shared_limit=shared_limit, threads=8)
    bound = layer_bound(oracle, sem, experts, shared, ids, w, x, H, F, routed_limit,
                        shared_limit)
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= bound), float((err / bound).max())
    return layer


@pytest.mark.parametrize("routing_name,score", [("learned", "sigmoid"), ("learned", "sqrt_softplus"),
                                                ("table", "sigmoid"), ("softmax", None)])
def test_small_layers(ops, lib, oracle, routing_name, score):
    print(f"[moe small] {routing_name} {score}", flush=True)
    rng = np.random.default_rng(42)
    from vastloom_amd.workloads import MoeWorkload
    sem = "qwen" if routing_name == "softmax" else "deepseek"
    wl = MoeWorkload("small", 11, 512, 256, 24, 4, 5, IQ2_XXS, IQ2_XXS, 0.01, sem)
    experts = [make_expert(rng, IQ2_XXS, IQ2_XXS, 512, 256) for _ in range(24)]
    shared = make_expert(rng, IQ2_XXS, IQ2_XXS, 512, 256)
    x = rng.standard_normal((5, 512)).astype(np.float32)
    bias = (rng.standard_normal(24) * 0.05).astype(np.float32) if routing_name == "learned" else None
    table = np.stack([rng.choice(24, 4, replace=False) for _ in range(5)]) if routing_name == "table" else None
    routing = {"learned": lib.ROUTE_LEARNED, "table": lib.ROUTE_TABLE,
               "softmax": lib.ROUTE_SOFTMAX}[routing_name]
    sf = SCORE_SQRT_SOFTPLUS if score == "sqrt_softplus" else SCORE_SIGMOID
    _check_layer(ops, lib, oracle, wl, experts, shared, sem, routing_name, routing, x, sf, bias,
                 table, route_scale=1.5 if sem == "deepseek" else 1.0,
                 routed_limit=0.3 if sem == "deepseek" else 0.0,
                 shared_limit=0.2 if sem == "deepseek" else 0.0)


@pytest.mark.parametrize("experts_n,tokens,routing_name", [(256, 1, "learned"), (100, 3, "learned"),
                                                         (64, 2, "softmax")])
def test_tied_router_rows_route_to_lower_ids(ops, lib, oracle, experts_n, tokens, routing_name):
    """Router rows repeated in runs of four give equal logits (and keys) within each run; the
    selection must take the runs' lower expert ids first, as the reference's stable ranking does."""
    print(f"[moe ties] E={experts_n} tokens={tokens} {routing_name}", flush=True)
    rng = np.random.default_rng(7 + experts_n)
    from vastloom_amd.workloads import MoeWorkload
    sem = "qwen" if routing_name == "softmax" else "deepseek"
    H, F, K = 256, 256, 6
    wl = MoeWorkload("ties", 13, H, F, experts_n, K, tokens, IQ2_XXS, IQ2_XXS, 0.01, sem)
    base = (rng.standard_normal(((experts_n + 3) // 4, H)) * 0.02).astype(np.float32)
    router = np.ascontiguousarray(np.repeat(base, 4, axis=0)[:experts_n])
    experts = [make_expert(rng, IQ2_XXS, IQ2_XXS, H, F) for _ in range(experts_n)]
    shared = make_expert(rng, IQ2_XXS, IQ2_XXS, H, F)
    x = rng.standard_normal((tokens, H)).astype(np.float32)
    routing = lib.ROUTE_SOFTMAX if routing_name == "softmax" else lib.ROUTE_LEARNED
    layer = _check_layer(ops, lib, oracle, wl, experts, shared, sem, routing_name, routing, x,
                         router=router)
    ids, _ = layer.routes(tokens)
    for t in range(tokens):  # every run the selection enters is entered at its lowest id
        for e in ids[t]:
            assert e % 4 == 0 or (e - 1) in ids[t], (t, ids[t])


@pytest.mark.parametrize("experts_n,tokens,routing_name", [(300, 1, "learned"), (600, 2, "softmax"),
                                                         (1024, 1, "learned")])
def test_wide_expert_pools(ops, lib, oracle, experts_n, tokens, routing_name):
    """Pools above 256 experts: the gate/up blocks take the experts' pointers from global memory
    instead of their LDS table, and the top-k keeps 8 or 16 keys per lane."""
    print(f"[moe wide] E={experts_n} tokens={tokens} {routing_name}", flush=True)
    rng = np.random.default_rng(11 + experts_n)
    from vastloom_amd.workloads import MoeWorkload
    sem = "qwen" if routing_name == "softmax" else "deepseek"
    H, F, K = 256, 256, 8
    wl = MoeWorkload("wide", 19, H, F, experts_n, K, tokens, IQ2_XXS, IQ2_XXS, 0.01, sem)
    experts = [make_expert(rng, IQ2_XXS, IQ2_XXS, H, F) for _ in range(experts_n)]
    shared = make_expert(rng, IQ2_XXS, IQ2_XXS, H, F) if sem == "deepseek" else None
    x = rng.standard_normal((tokens, H)).astype(np.float32)
    routing = lib.ROUTE_SOFTMAX if routing_name == "softmax" else lib.ROUTE_LEARNED
    _check_layer(ops, lib, oracle, wl, experts, shared, sem, routing_name, routing, x)


@pytest.mark.parametrize("experts_n,top_k,tokens,routing_name", [
    (64, 12, 1, "learned"), (64, 16, 1, "softmax"), (48, 16, 3, "learned"), (64, 12, 20, "learned"),
    (40, 16, 9, "softmax")])
def test_wide_top_k(ops, lib, oracle, experts_n, top_k, tokens, routing_name):
    """top_k 12 and 16 (the header's limit), single token, token slots and the grouped path."""
    print(f"[moe top_k] E={experts_n} K={top_k} tokens={tokens} {routing_name}", flush=True)
    rng = np.random.default_rng(100 + experts_n + top_k + tokens)
    from vastloom_amd.workloads import MoeWorkload
    sem = "qwen" if routing_name == "softmax" else "deepseek"
    H, F = 512, 256
    wl = MoeWorkload("topk", 21, H, F, experts_n, top_k, tokens, IQ2_XXS, IQ2_XXS, 0.01, sem)
    experts = [make_expert(rng, IQ2_XXS, IQ2_XXS, H, F) for _ in range(experts_n)]
    shared = make_expert(rng, IQ2_XXS, IQ2_XXS, H, F) if sem == "deepseek" else None
    x = rng.standard_normal((tokens, H)).astype(np.float32)
    bias = (rng.standard_normal(experts_n) * 0.05).astype(np.float32) if routing_name == "learned" else None
    routing = lib.ROUTE_SOFTMAX if routing_name == "softmax" else lib.ROUTE_LEARNED
    _check_layer(ops, lib, oracle, wl, experts, shared, sem, routing_name, routing, x, SCORE_SIGMOID,
                 bias, route_scale=1.25 if sem == "deepseek" else 1.0)


def test_bad_table_route_is_refused(ops, lib, oracle):
    rng = np.random.default_rng(1)
    from vastloom_amd.workloads import MoeWorkload
    wl = MoeWorkload("bad", 12, 256, 256, 4, 2, 1, IQ2_XXS, IQ2_XXS, 0.01, "deepseek")
    experts = [make_expert(rng, IQ2_XXS, IQ2_XXS, 256, 256) for _ in range(4)]
    layer = _device_layer(ops, lib, wl, experts, None, "deepseek", lib.ROUTE_TABLE, wl.router())
    x = torch.from_numpy(rng.standard_normal((1, 256)).astype(np.float32)).cuda()
    for bad in ([[1, 7]], [[2, 2]]):
        with pytest.raises(ops.VlError):
            layer.forward(x, table_ids=torch.tensor(bad, dtype=torch.int32).cuda())


@pytest.mark.parametrize("tokens", [1, 3, 20])
@pytest.mark.parametrize("case", ["bias", "table_logit"])
def test_nonfinite_routing_inputs_are_refused(ops, lib, oracle, tokens, case):
    """A non-finite selection bias (learned routing), or a non-finite logit of an expert the table
    does not select, refuses the layer, as the reference's require_finite of the bias and the
    logits does (deepseek_v4_reference.cpp:235-238, :161): single-token, token-slot and grouped
    paths."""
    print(f"[moe refuse] {case} tokens={tokens}", flush=True)
    rng = np.random.default_rng(7 + tokens)
    from vastloom_amd.workloads import MoeWorkload
    H, F, E, K = 256, 256, 6, 2
    wl = MoeWorkload("refuse", 15, H, F, E, K, tokens, IQ2_XXS, IQ2_XXS, 0.01, "deepseek")
    experts = [make_expert(rng, IQ2_XXS, IQ2_XXS, H, F) for _ in range(E)]
    router = wl.router()
    x = torch.from_numpy(rng.standard_normal((tokens, H)).astype(np.float32)).cuda()
    if case == "bias":
        bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
        ok = _device_layer(ops, lib, wl, experts, None, "deepseek", lib.ROUTE_LEARNED, router, bias)
        assert torch.isfinite(ok.forward(x)).all()
        bias[E - 1] = np.inf
        bad = _device_layer(ops, lib, wl, experts, None, "deepseek", lib.ROUTE_LEARNED, router, bias)
        with pytest.raises(ops.VlError):
            bad.forward(x)
    else:
        table = torch.from_numpy(np.tile(np.array([[0, 1]], np.uint32), (tokens, 1))).cuda()
        ok = _device_layer(ops, lib, wl, experts, None, "deepseek", lib.ROUTE_TABLE, router)
        assert torch.isfinite(ok.forward(x, table_ids=table)).all()
        router = router.copy()
        router[E - 1, 0] = np.nan  # expert E-1's logit, which the table never selects
        bad = _device_layer(ops, lib, wl, experts, None, "deepseek", lib.ROUTE_TABLE, router)
        with pytest.raises(ops.VlError):
            bad.forward(x, table_ids=table)


def _workload_case(wl):
    experts = [wl.expert(e).triple() for e in range(wl.experts)]
    shared = wl.shared().triple() if wl.has_shared else None
    return experts, shared


def test_workload_q8_expert(ops, lib, oracle):
    wl = workload("q8_expert")
    print("[workload] q8_expert", flush=True)
    triple = wl.expert(0).triple()
    x = wl.x()
    want = oracle.expert_qwen(*triple, wl.width, wl.intermediate, x[0], threads=8)
    got = ops.expert_ffn(device_expert(ops, triple, wl.width, wl.intermediate),
                         torch.from_numpy(x).cuda(), semantics=1).cpu().numpy()[0]
    h = expert_h(oracle, "qwen", triple, wl.width, wl.intermediate, x[0])
    bound = TOL * down_row_norms(oracle, triple, wl.width, wl.intermediate) * np.linalg.norm(h)
    assert np.all(np.abs(got.astype(np.float64) - want) <= bound)


def test_workload_q8_moe(ops, lib, oracle):
    wl = workload("q8_moe")
    print("[workload] q8_moe", flush=True)
    experts, shared = _workload_case(wl)
    _check_layer(ops, lib, oracle, wl, experts, shared, "qwen", "softmax", lib.ROUTE_SOFTMAX,
                 wl.x())


@pytest.mark.parametrize("name", ["iq2_moe", "mixed_moe"])
def test_workload_deepseek_layers(ops, lib, oracle, name):
    wl = workload(name)
    print(f"[workload] {name}", flush=True)
    experts, shared = _workload_case(wl)
    _check_layer(ops, lib, oracle, wl, experts, shared, "deepseek", "learned", lib.ROUTE_LEARNED,
                 wl.x(), SCORE_SIGMOID)


# -- Grouped path: more than 8 tokens -------------------------------------------------------------

@pytest.mark.parametrize("routing_name,tokens,gt,dt", [
    ("learned", 9, IQ2_XXS, IQ2_XXS), ("table", 37, IQ2_XXS, IQ2_XXS),
    ("softmax", 100, Q8_0, Q8_0), ("learned", 64, IQ1_S, IQ3_XXS),
    ("learned", 1024, IQ2_XXS, IQ2_XXS)])
def test_grouped_layers(ops, lib, oracle, routing_name, tokens, gt, dt):
    print(f"[moe grouped] {routing_name} tokens={tokens} types={gt},{dt}", flush=True)
    rng = np.random.default_rng(tokens)
    from vastloom_amd.workloads import MoeWorkload
    sem = "qwen" if routing_name == "softmax" else "deepseek"
    E, K, H, F = 24, 4, 512, 256
    wl = MoeWorkload("grouped_small", 13, H, F, E, K, tokens, gt, dt, 0.01, sem)
    experts = [make_expert(rng, gt, dt, H, F) for _ in range(E)]
    shared = make_expert(rng, gt, dt, H, F)
    x = rng.standard_normal((tokens, H)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32) if routing_name == "learned" else None
    table = (np.stack([rng.choice(E, K, replace=False) for _ in range(tokens)])
             if routing_name == "table" else None)
    routing = {"learned": lib.ROUTE_LEARNED, "table": lib.ROUTE_TABLE,
               "softmax": lib.ROUTE_SOFTMAX}[routing_name]
    _check_layer(ops, lib, oracle, wl, experts, shared, sem, routing_name, routing, x,
                 SCORE_SIGMOID, bias, table, route_scale=1.5 if sem == "deepseek" else 1.0,
                 routed_limit=0.3 if sem == "deepseek" else 0.0,
                 shared_limit=0.2 if sem == "deepseek" else 0.0)


def test_grouped_bad_route_is_refused(ops, lib, oracle):
    rng = np.random.default_rng(2)
    from vastloom_amd.workloads import MoeWorkload
    wl = MoeWorkload("grouped_bad", 14, 256, 256, 6, 2, 20, IQ2_XXS, IQ2_XXS, 0.01, "deepseek")
    experts = [make_expert(rng, IQ2_XXS, IQ2_XXS, 256, 256) for _ in range(6)]
    layer = _device_layer(ops, lib, wl, experts, None, "deepseek", lib.ROUTE_TABLE, wl.router())
    x = torch.from_numpy(rng.standard_normal((20, 256)).astype(np.float32)).cuda()
    table = np.stack([rng.choice(6, 2, replace=False) for _ in range(20)]).astype(np.int32)
    ok = layer.forward(x, table_ids=torch.from_numpy(table).cuda())
    assert torch.isfinite(ok).all()
    table[13] = [4, 4]
    with pytest.raises(ops.VlError):
        layer.forward(x, table_ids=torch.from_numpy(table).cuda())


def test_workload_grouped_moe(ops, lib, oracle):
    """512 tokens, Zipf(1.1) table routing over 256 IQ2_XXS experts plus the shared expert:
    every token's routes, and the outputs of 69 sampled tokens, against the oracle."""
    wl = workload("grouped_moe")
    print("[workload] grouped_moe", flush=True)
    experts, shared = _workload_case(wl)
    # A seeded sample of 64 tokens plus the ends and the middle (each token's output depends on
    # its own routes only; all 512 tokens' routes are checked).
    sample = np.union1d(np.random.default_rng(4).choice(512, 64, replace=False), [0, 1, 255, 256, 511])
    _check_layer(ops, lib, oracle, wl, experts, shared, "deepseek", "table", lib.ROUTE_TABLE,
                 wl.x(), SCORE_SIGMOID, table=wl.zipf_table(), sample=sample)


@pytest.mark.parametrize("routing_name,tokens,gt,dt", [
    ("learned", 1, Q4_K, Q6_K), ("learned", 5, IQ2_XXS, MXFP4), ("table", 20, Q5_K, Q5_K),
    ("softmax", 3, MXFP4, MXFP4), ("learned", 2, IQ2_S, Q4_K)])
def test_gguf_layout_layers(ops, lib, oracle, routing_name, tokens, gt, dt):
    # Layers whose experts (shared expert included) are K-quant, IQ2_S or MXFP4 matrices run on
    # the grouped plan at every token count; routes and outputs as for the other layers.
    print(f"[moe gguf] {routing_name} tokens={tokens} {gt}/{dt}", flush=True)
    rng = np.random.default_rng(700 + tokens + gt + dt)
    from vastloom_amd.workloads import MoeWorkload
    sem = "qwen" if routing_name == "softmax" else "deepseek"
    H, F, E, K = 1024, 512, 16, 4
    wl = MoeWorkload("gguf", 13, H, F, E, K, tokens, gt, dt, 0.01, sem)
    experts = [make_expert(rng, gt, dt, H, F) for _ in range(E)]
    shared = make_expert(rng, gt, dt, H, F)
    x = rng.standard_normal((tokens, H)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32) if routing_name == "learned" else None
    table = np.stack([rng.choice(E, K, replace=False) for _ in range(tokens)]) if routing_name == "table" else None
    routing = {"learned": lib.ROUTE_LEARNED, "table": lib.ROUTE_TABLE,
               "softmax": lib.ROUTE_SOFTMAX}[routing_name]
    _check_layer(ops, lib, oracle, wl, experts, shared, sem, routing_name, routing, x, SCORE_SIGMOID,
                 bias, table, route_scale=1.5 if sem == "deepseek" else 1.0,
                 routed_limit=0.3 if sem == "deepseek" else 0.0,
                 shared_limit=0.2 if sem == "deepseek" else 0.0)

