"""The oracle against the reference's own CPU kernels, compiled from its sources (no GPU).

oracle/_ref/libvlref.so is built by `make -C oracle ref` from the reference tree; where it is
absent these tests skip. Decoders, matvecs, the fused IQ1_S/IQ3_XXS expert and the Q8_0 expert
MLP must be bit-identical; routing must select the same experts with bit-identical weights.
Shapes include the workload shapes (OLMoE-sized Q8_0 experts, DeepSeek-sized IQ matrices).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle.oracle import (BF16, IQ1_S, IQ2_S, IQ2_XXS, IQ3_XXS, MXFP4, Q4_K, Q5_K, Q6_K, Q8_0,
                           SCORE_SQRT_SOFTPLUS, OracleError)
from vastloom_amd.workloads import random_matrix, workload

SHAPES = {
    Q8_0: [(3, 64), (64, 2048), (1024, 2048), (2048, 1024)],
    IQ2_XXS: [(3, 512), (130, 1024), (2048, 7168), (7168, 2048)],
    IQ3_XXS: [(3, 512), (65, 2048), (512, 2048)],
    IQ1_S: [(3, 512), (64, 1792), (256, 7168)],
    Q4_K: [(3, 512), (130, 2048), (2048, 7168)],
    Q5_K: [(3, 512), (65, 2048), (512, 7168)],
    Q6_K: [(3, 512), (64, 1792), (1024, 2048)],
    MXFP4: [(3, 64), (45, 2880), (512, 2048)],
    IQ2_S: [(3, 512), (65, 2048), (512, 7168)],
    BF16: [(2, 4), (33, 100), (512, 2048)],
}


@pytest.mark.parametrize("qtype,rows,cols",
                         [(t, r, c) for t, shapes in SHAPES.items() for r, c in shapes])
def test_decode_and_matvec_bit_identical(oracle, reference, qtype, rows, cols):
    rng = np.random.default_rng(rows * 131 + cols + qtype)
    enc = random_matrix(rng, qtype, rows, cols, 0.01)
    n = rows * cols
    if n <= 4_000_000:
        assert np.array_equal(oracle.dequantize(qtype, enc, n).view(np.uint32),
                              reference.dequantize(qtype, enc, n).view(np.uint32))
    x = rng.standard_normal(cols).astype(np.float32)
    for threads in (1, 4):
        a = oracle.matvec(qtype, enc, rows, cols, x, threads=threads)
        b = reference.matvec(qtype, enc, rows, cols, x, threads=threads)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_subnormal_and_extreme_scales_bit_identical(oracle, reference):
    # fp16 subnormal, smallest normal and largest finite scales in every format.
    rng = np.random.default_rng(3)
    for qtype, (rows, cols) in ((Q8_0, (8, 256)), (IQ2_XXS, (8, 512)), (IQ3_XXS, (8, 512)),
                                (IQ1_S, (8, 512)), (IQ2_S, (8, 512))):
        enc = random_matrix(rng, qtype, rows, cols, 0.01)
        bb = enc.size // (rows * cols // (32 if qtype == Q8_0 else 256))
        blocks = enc.reshape(-1, bb)
        special = np.array([0x0001, 0x03FF, 0x0400, 0x7BFF, 0x8001, 0xFBFF, 0x0000], np.uint16)
        s = special[np.arange(blocks.shape[0]) % special.size]
        blocks[:, 0], blocks[:, 1] = s & 0xFF, s >> 8
        n = rows * cols
        assert np.array_equal(oracle.dequantize(qtype, enc, n).view(np.uint32),
                              reference.dequantize(qtype, enc, n).view(np.uint32))
        x = rng.standard_normal(cols).astype(np.float32) * 1e-3
        a = oracle.matvec(qtype, enc, rows, cols, x)
        b = reference.matvec(qtype, enc, rows, cols, x)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_routed_expert_iq1s_iq3xxs_bit_identical(oracle, reference):
    rng = np.random.default_rng(17)
    H, F = 1024, 512
    gate = random_matrix(rng, IQ1_S, F, H, 0.01)
    up = random_matrix(rng, IQ1_S, F, H, 0.01)
    down = random_matrix(rng, IQ3_XXS, H, F, 0.01)
    x = rng.standard_normal(H).astype(np.float32)
    a = oracle.routed_expert_iq1s_iq3xxs(gate, up, down, H, F, x)
    b = reference.routed_expert_iq1s_iq3xxs(gate, up, down, H, F, x)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_q8_expert_mlp_bit_identical_at_workload_shape(oracle, reference):
    wl = workload("q8_expert")
    e = wl.expert(0)
    x = wl.x()[0]
    a = oracle.expert_qwen((Q8_0, e.gate), (Q8_0, e.up), (Q8_0, e.down), wl.width,
                           wl.intermediate, x, threads=4)
    b = reference.qwen_expert_mlp_q8(e.gate, e.up, e.down, wl.width, wl.intermediate, x)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("tokens,experts,top_k", [(1, 256, 8), (5, 256, 8), (7, 64, 6)])
def test_routes_bit_identical(oracle, reference, tokens, experts, top_k):
    rng = np.random.default_rng(tokens * experts)
    logits = (rng.standard_normal((tokens, experts)) * 1.7).astype(np.float32)
    bias = (rng.standard_normal(experts) * 0.05).astype(np.float32)
    a = oracle.route_learned(logits, bias, top_k, 2.5, SCORE_SQRT_SOFTPLUS)
    b = reference.route_learned(logits, bias, top_k, 2.5)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1].view(np.uint32), b[1].view(np.uint32))
    table = np.stack([rng.choice(experts, top_k, replace=False) for _ in range(11)]).astype(np.uint32)
    ids = rng.integers(0, 11, tokens).astype(np.uint32)
    a = oracle.route_hash(logits, ids, table, top_k, 1.0, SCORE_SQRT_SOFTPLUS)
    b = reference.route_hash(logits, ids, table, top_k, 1.0)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1].view(np.uint32), b[1].view(np.uint32))


def test_qwen_route_bit_identical_at_workload_shape(oracle, reference):
    wl = workload("q8_moe")
    router, x = wl.router(), wl.x()[0]
    idx_r, w_r, logits_r = reference.qwen_route(x, router, wl.experts, wl.top_k, True)
    logits = oracle.linear_f64(router, x, wl.experts)[0]
    assert np.array_equal(logits.view(np.uint32), logits_r.view(np.uint32))
    idx, w = oracle.route_softmax(logits, wl.top_k, True)
    assert np.array_equal(idx, idx_r) and np.array_equal(w.view(np.uint32), w_r.view(np.uint32))


def test_clamped_expert_against_reference_float_oracle(oracle, reference):
    # deepseek_v4_expert_swiglu keeps gate/up in float64 where execute_expert rounds them to
    # float first, so the two agree to float rounding, not bit for bit.
    rng = np.random.default_rng(23)
    H, F, T = 256, 64, 3
    g = (rng.standard_normal((F, H)) * 0.1).astype(np.float32)
    u = (rng.standard_normal((F, H)) * 0.1).astype(np.float32)
    d = (rng.standard_normal((H, F)) * 0.1).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    route = np.array([0.3, 1.1, 0.7], np.float32)
    for limit in (0.0, 0.5):
        a = oracle.expert_deepseek((0, g.view(np.uint8)), (0, u.view(np.uint8)),
                                   (0, d.view(np.uint8)), H, F, x, routing=route, limit=limit)
        b = reference.expert_swiglu_f32(x, g, d, u, route, H, F, limit)
        assert np.allclose(a, b, atol=1e-6 * np.abs(b).max(), rtol=0)


def _outcome(fn):
    try:
        return fn()
    except OracleError as e:  # both wrappers raise it with the reference's error code
        return e.name


@pytest.mark.parametrize("qtype", [Q4_K, Q5_K, Q6_K])
def test_k_quant_special_scales_bit_identical(oracle, reference, qtype):
    # fp16 subnormal, smallest normal, largest finite, negative and zero d / dmin, then an
    # infinite and a NaN one, which both sides must refuse alike.
    rng = np.random.default_rng(qtype)
    rows, cols = 7, 512
    special = np.array([0x0001, 0x03FF, 0x0400, 0x7BFF, 0x8001, 0xFBFF, 0x0000], np.uint16)
    offsets = (208,) if qtype == Q6_K else (0, 2)
    enc = random_matrix(rng, qtype, rows, cols, 0.01)
    blocks = enc.reshape(rows * cols // 256, -1)
    for i, off in enumerate(offsets):
        s = special[(np.arange(blocks.shape[0]) + 3 * i) % special.size]
        blocks[:, off], blocks[:, off + 1] = s & 0xFF, s >> 8
    n = rows * cols
    x = rng.standard_normal(cols).astype(np.float32)
    assert np.array_equal(oracle.dequantize(qtype, enc, n).view(np.uint32),
                          reference.dequantize(qtype, enc, n).view(np.uint32))
    assert np.array_equal(oracle.matvec(qtype, enc, rows, cols, x).view(np.uint32),
                          reference.matvec(qtype, enc, rows, cols, x).view(np.uint32))
    for bad_bits in (0x7C00, 0xFE00):
        for off in offsets:
            bad = enc.copy().reshape(blocks.shape)
            bad[5, off], bad[5, off + 1] = bad_bits & 0xFF, bad_bits >> 8
            bad = bad.reshape(-1)
            a = _outcome(lambda: oracle.dequantize(qtype, bad, n))
            b = _outcome(lambda: reference.dequantize(qtype, bad, n))
            assert a == b == "invalid_format"
            a = _outcome(lambda: oracle.matvec(qtype, bad, rows, cols, x))
            b = _outcome(lambda: reference.matvec(qtype, bad, rows, cols, x))
            assert a == b == "invalid_format"


def test_mxfp4_every_scale_byte(oracle, reference):
    # All 256 E8M0 scale bytes against all 256 code bytes: the subnormal scales 0 and 1, the
    # normal range, and the top bytes whose large codes overflow to infinity (refused by both).
    codes = np.arange(256, dtype=np.uint8)
    for e in range(256):
        enc = np.zeros((16, 17), np.uint8)
        enc[:, 0] = e
        enc[:, 1:] = codes.reshape(16, 16)
        enc = enc.reshape(-1)
        a = _outcome(lambda: oracle.dequantize(MXFP4, enc, 512))
        b = _outcome(lambda: reference.dequantize(MXFP4, enc, 512))
        if isinstance(a, str) or isinstance(b, str):
            assert a == b == "invalid_format", e
        else:
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), e
            assert np.all(np.isfinite(a))
    x = np.linspace(-1, 1, 64).astype(np.float32)
    enc = random_matrix(np.random.default_rng(39), MXFP4, 16, 64, 0.01)
    enc.reshape(-1, 17)[:, 0] = np.arange(32) % 2  # the two subnormal scales
    assert np.array_equal(oracle.matvec(MXFP4, enc, 16, 64, x).view(np.uint32),
                          reference.matvec(MXFP4, enc, 16, 64, x).view(np.uint32))


def test_bf16_special_values(oracle, reference):
    # Every finite bf16 bit pattern decodes alike; an infinity or NaN anywhere is refused alike.
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = np.isfinite((codes.astype(np.uint32) << 16).view(np.float32))
    enc = codes[finite].view(np.uint8)
    n = int(finite.sum())
    a = oracle.dequantize(BF16, enc, n)
    assert np.array_equal(a.view(np.uint32), reference.dequantize(BF16, enc, n).view(np.uint32))
    assert np.array_equal(a.view(np.uint32), codes[finite].astype(np.uint32) << 16)
    for bad_code in (0x7F80, 0xFF80, 0x7FC1):
        bad = np.array([0x3F80, bad_code, 0x4000, 0x3F00], np.uint16).view(np.uint8)
        x = np.ones(2, np.float32)
        assert _outcome(lambda: oracle.dequantize(BF16, bad, 4)) == "invalid_format"
        assert _outcome(lambda: reference.dequantize(BF16, bad, 4)) == "invalid_format"
        assert _outcome(lambda: oracle.matvec(BF16, bad, 2, 2, x)) == \
            _outcome(lambda: reference.matvec(BF16, bad, 2, 2, x))
