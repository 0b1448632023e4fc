"""vl_moe_layer_noalloc (the entry point that allocates nothing) against vl_moe_layer, through
the C ABI: the same layer computed with the library's static per-device workspace must give the
same outputs, bit for bit, as with a caller-owned workspace, on two calls in a row where the
second call is smaller than the first (the static workspace keeps the first call's contents)."""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
import torch

from oracle.oracle import IQ2_XXS, SCORE_SIGMOID
from vastloom_amd.workloads import random_matrix

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    assert torch.cuda.is_available(), "GPU tests need a visible HIP device"
    from vastloom_amd import _lib, ops

    return ops, _lib


def build_layer(ops, _lib, rng, H=1024, F=512, E=16, K=4):
    def expert():
        return ops.DeviceExpert(IQ2_XXS, IQ2_XXS, H, F, random_matrix(rng, IQ2_XXS, F, H, 0.01),
                                random_matrix(rng, IQ2_XXS, F, H, 0.01),
                                random_matrix(rng, IQ2_XXS, H, F, 0.01))

    experts = [expert() for _ in range(E)]
    shared = expert()
    router = torch.from_numpy((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    bias = torch.from_numpy((rng.standard_normal(E) * 0.01).astype(np.float32))
    return ops.MoeLayer(experts, shared, width=H, intermediate=F, top_k=K, gate_type=IQ2_XXS,
                        down_type=IQ2_XXS, semantics=0, routing=_lib.ROUTE_LEARNED,
                        score_fn=SCORE_SIGMOID, routed_limit=0.5, shared_limit=0.5,
                        router=router, bias=bias)


def noalloc_forward(_lib, layer, x):
    tokens = x.shape[0]
    out = torch.full_like(x, float("nan"))
    cfg = layer.config(tokens)
    inputs = _lib.MoeInputs(layer.expert_table.data_ptr(), layer.router.data_ptr(),
                            layer.bias.data_ptr(), 0, 0, 0, x.data_ptr(), out.data_ptr())
    stream = torch.cuda.current_stream().cuda_stream
    rc = _lib.lib().vl_moe_layer_noalloc(C.byref(cfg), C.byref(inputs), C.c_void_p(stream))
    assert rc == 0, _lib.lib().vl_last_error()
    bits = C.c_uint32(0xffffffff)
    assert _lib.lib().vl_moe_noalloc_status(C.c_void_p(stream), C.byref(bits)) == 0
    assert bits.value == 0, bits.value
    return out


def test_noalloc_matches_caller_workspace_on_two_calls(env):
    ops, _lib = env
    rng = np.random.default_rng(21)
    layer = build_layer(ops, _lib, rng)
    for tokens in (5, 1):  # the second call is smaller than the first
        print(f"[noalloc] tokens={tokens}", flush=True)
        x = torch.from_numpy(rng.standard_normal((tokens, layer.width)).astype(np.float32)).cuda()
        want = layer.forward(x).cpu().numpy()
        got = noalloc_forward(_lib, layer, x).cpu().numpy()
        assert np.all(np.isfinite(got))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_noalloc_refuses_layers_beyond_its_workspace(env):
    ops, _lib = env
    # A 1024-token prefill at the DeepSeek shape needs far more than the static workspace; it is
    # refused before anything is launched (no weights are read, so null expert pointers are fine).
    cfg = _lib.MoeConfig(1024, 7168, 2048, 256, 8, IQ2_XXS, IQ2_XXS, 0, _lib.ROUTE_LEARNED,
                         SCORE_SIGMOID, 1, 1, 1.0, 0.0, 0.0)
    dummy = 256
    inputs = _lib.MoeInputs(dummy, dummy, 0, 0, 0, 0, dummy, dummy)
    rc = _lib.lib().vl_moe_layer_noalloc(C.byref(cfg), C.byref(inputs), None)
    assert rc == 9, rc  # resource_exhausted
    assert b"static workspace" in _lib.lib().vl_last_error()
