"""The oracle against the reference's committed known-answer vectors (no GPU).

Mirrors test_trunk_storage_reference_kernels, test_iq1_s_reference_kernel,
test_iq2_xxs_reference_kernel, test_q4k_mxfp4_reference_parity, test_iq3_xxs_reference_kernel,
test_quantized_routed_expert_contract and test_qwen38_moe_router
(reference tests/test_main.cpp:863-1112, :1295-1460, :1663-1723, :1832-1907, :2006-2051,
:3966-3990).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle.oracle import IQ1_S, IQ2_XXS, IQ3_XXS, Q8_0, OracleError
from tests.kat_blocks import KAT, fnv_f32, kat_count, kat_poisoned, kat_rows, kat_x


def test_codebook_fingerprints(oracle):
    # The compact codebooks expand to tables whose FNV-1a fingerprints are the reference's
    # compile-time pins (ggml_quantization.cpp:60,73,99).
    assert oracle.codebooks_ok()


def test_fp16_decode_exhaustive(oracle):
    # Every binary16 code, subnormals, infinities and NaN payloads included, against numpy's
    # exact widening conversion.
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    expected = codes.view(np.float16).astype(np.float32).view(np.uint32)
    got = np.array([oracle.fp16_to_f32(int(c)) for c in codes], np.float32).view(np.uint32)
    finite = np.isfinite(codes.view(np.float16))
    assert np.array_equal(got[finite], expected[finite])
    # Infinities keep their sign; NaN codes stay NaN (the float return through ctypes quiets a
    # signalling payload, so only the class is compared; every decoder refuses them anyway).
    g, e = got[~finite].view(np.float32), expected[~finite].view(np.float32)
    assert np.array_equal(np.isnan(g), np.isnan(e))
    assert np.array_equal(g[~np.isnan(e)], e[~np.isnan(e)])


@pytest.mark.parametrize("name", sorted(KAT))
def test_decode_fingerprint_and_values(oracle, name):
    k = KAT[name]
    enc = k["blocks"]()
    out = oracle.dequantize(k["qtype"], enc, kat_count(k))
    if k["fnv"] is not None:
        assert fnv_f32(out) == k["fnv"]
    for index, value in k["values"].items():
        assert out[index] == np.float32(value), (name, index)
    for index, (value, tol) in k.get("approx", {}).items():
        assert abs(float(out[index]) - value) <= tol, (name, index)


@pytest.mark.parametrize("name", sorted(KAT))
@pytest.mark.parametrize("threads", [1, 4])
def test_matvec_known_outputs(oracle, name, threads):
    k = KAT[name]
    cols = k["cols"]
    y = oracle.matvec(k["qtype"], k["blocks"](), kat_rows(k), cols, kat_x(k), threads=threads)
    for got, (want, tol) in zip(y, k["outputs"]):
        if tol == 0.0:
            assert got == np.float32(want)
        else:
            assert abs(float(got) - want) <= tol


def test_dequantize_row_matches_full_decode(oracle):
    k = KAT["iq2_xxs"]
    enc = k["blocks"]()
    full = oracle.dequantize(IQ2_XXS, enc, 6 * 256)
    assert np.array_equal(oracle.dequantize_row(IQ2_XXS, enc, 3, 512, 1), full[512:1024])
    with pytest.raises(OracleError):
        oracle.dequantize_row(IQ2_XXS, enc, 3, 512, 3)


@pytest.mark.parametrize("name", sorted(KAT))
def test_malformed_inputs_fail_closed(oracle, name):
    k = KAT[name]
    qtype, be = k["qtype"], k["block_elements"]
    enc = k["blocks"]()
    cols, rows = k["cols"], kat_rows(k)
    x = kat_x(k)
    n = kat_count(k)
    sentinel = np.full(n, 17.0, np.float32)
    # Truncated payload, empty output, a ceiling below the matrix, an unaligned column count.
    with pytest.raises(OracleError):
        oracle.dequantize(qtype, enc[:-1], n, out=sentinel)
    with pytest.raises(OracleError):
        oracle.dequantize(qtype, enc, 0)
    with pytest.raises(OracleError):
        oracle.dequantize(qtype, enc, n, max_elements=be)
    with pytest.raises(OracleError):
        oracle.matvec(qtype, enc, rows, cols - 1, x[:-1])
    with pytest.raises(OracleError):
        oracle.matvec(qtype, enc[:-1], rows, cols, x)
    assert np.all(sentinel == 17.0)
    # A non-finite block scale (or value) is refused and the destination is left untouched.
    bad = kat_poisoned(k)
    with pytest.raises(OracleError) as err:
        oracle.dequantize(qtype, bad, n, out=sentinel)
    assert err.value.name == "invalid_format"
    assert np.all(sentinel == 17.0)
    ys = np.full(rows, 17.0, np.float32)
    with pytest.raises(OracleError):
        oracle.matvec(qtype, bad, rows, cols, x, out=ys)
    assert np.all(ys == 17.0)
    # A NaN input is refused.
    xn = x.copy()
    xn[0] = np.nan
    with pytest.raises(OracleError) as err:
        oracle.matvec(qtype, enc, rows, cols, xn, out=ys)
    assert err.value.name == "invalid_argument"
    assert np.all(ys == 17.0)


def test_routed_expert_contract(oracle):
    # All-zero IQ1_S gate/up and IQ3_XXS down blocks decode to zero weights, so the expert
    # output is exactly zero (test_main.cpp:2006-2020).
    dim = 256
    gate = np.zeros(dim * 50, np.uint8)
    up = np.zeros(dim * 50, np.uint8)
    down = np.zeros(dim * 98, np.uint8)
    x = np.full(dim, 0.25, np.float32)
    y = oracle.routed_expert_iq1s_iq3xxs(gate, up, down, dim, dim, x)
    assert np.all(y == 0.0)
    with pytest.raises(OracleError):
        oracle.routed_expert_iq1s_iq3xxs(gate[:-1], up, down, dim, dim, x)
    bad = down.copy()
    bad[0], bad[1] = 0x00, 0x7C
    with pytest.raises(OracleError):
        oracle.routed_expert_iq1s_iq3xxs(gate, up, bad, dim, dim, x)
    xn = x.copy()
    xn[0] = np.nan
    with pytest.raises(OracleError):
        oracle.routed_expert_iq1s_iq3xxs(gate, up, down, dim, dim, xn)


def test_qwen_softmax_router_known_answer(oracle):
    # hidden [1, 0] against router rows [1,0], [0,1], [1,1]: logits 1, 0, 1; the tie between
    # experts 0 and 2 keeps both, renormalised to one half each (test_main.cpp:3966-3990).
    hidden = np.array([1.0, 0.0], np.float32)
    router = np.array([1, 0, 0, 1, 1, 1], np.float32)
    logits = oracle.linear_f64(router, hidden, 3)[0]
    assert np.allclose(logits, [1.0, 0.0, 1.0], atol=1e-6)
    idx, w = oracle.route_softmax(logits, 2, True)
    assert list(idx) == [0, 2]
    assert np.allclose(w, [0.5, 0.5], atol=1e-5)
    with pytest.raises(OracleError):
        oracle.route_softmax(logits, 4, True)
