"""The CPU oracle reproduces the reference's own outputs bit for bit.

Fixtures: tests/golden/reference_vectors.npz, written by
tests/golden/make_golden.py from the reference sources compiled where they
lie (quants.c, kernels.c, gemma2.c mm). Every comparison is exact equality.
"""
import os

import numpy as np
import pytest

from oracle_lib import N_EMBD, Q8, dequantize_q8_0, fptr, gemm_q8_0, oracle, quantize_q8_0, vptr

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_vectors.npz")


@pytest.fixture(scope="module")
def g():
    return np.load(FIX, allow_pickle=False)


def q8(u8, rows):
    return np.ascontiguousarray(u8).view(Q8).reshape(rows, -1)


def test_fp16_conversion(g):
    o = oracle()
    got = np.array([o.or_fp32_to_fp16(float(v)) for v in g["fp16_in"]], dtype=np.uint16)
    assert np.array_equal(got, g["fp16_out"])


def test_fp16_to_fp32_is_exact():
    o = oracle()
    bits = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([o.or_fp16_to_fp32(int(b)) for b in bits], dtype=np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)]))
    assert np.array_equal(got[np.isinf(want)], want[np.isinf(want)])


def test_quantize_row(g):
    got = quantize_q8_0(g["quant_in"])
    assert np.array_equal(got.view(np.uint8).reshape(g["quant_out"].shape), g["quant_out"])


def test_rms_norm_family(g):
    o = oracle()
    x, w, h = g["norm_x"], g["norm_w"], g["norm_h"]
    for i in range(x.shape[0]):
        out = np.zeros(N_EMBD, np.float32)
        o.or_rms_norm(fptr(x[i]), fptr(w), N_EMBD, 1e-6, fptr(out))
        assert np.array_equal(out, g["norm_out"][i])
        blocks = np.zeros(24, dtype=Q8)
        o.or_rms_norm_quantize_q8_0(fptr(x[i]), fptr(w), N_EMBD, 1e-6, vptr(blocks))
        assert np.array_equal(blocks.view(np.uint8), g["norm_q8"][i])
        res = x[i].copy()
        o.or_rms_norm_residual_inplace(fptr(res), fptr(h[i]), fptr(w), N_EMBD, 1e-6)
        assert np.array_equal(res, g["resid_out"][i])


def test_qk_norm_rope(g):
    o = oracle()
    for i, (p, base) in enumerate(zip(g["qk_pos"], g["qk_base"])):
        q, k = g["qk_q_in"][i].copy(), g["qk_k_in"][i].copy()
        o.or_qk_norm_rope_qk_inplace(fptr(q), fptr(k), fptr(g["qk_qw"]), fptr(g["qk_kw"]), int(p), float(base), 1e-6)
        assert np.array_equal(q, g["qk_q_out"][i])
        assert np.array_equal(k, g["qk_k_out"][i])


@pytest.mark.parametrize("window,key", [(0, "att_full"), (8, "att_win8")])
def test_attention(g, window, key):
    o = oracle()
    T = g["att_q"].shape[0]
    ctx = np.zeros((T, N_EMBD), np.float32)
    sc = np.zeros(4096, np.float32)
    o.or_attention_range(fptr(g["att_q"]), fptr(g["att_k"]), fptr(g["att_v"]), T, window, 0, T, fptr(ctx), fptr(sc))
    assert np.array_equal(ctx, g[key])


def test_gelu(g):
    o = oracle()
    got = np.array([o.or_gelu_tanh(float(v)) for v in g["gelu_in"]], np.float32)
    assert np.array_equal(got, g["gelu_out"])
    for i in range(g["geglu_gate"].shape[0]):
        blocks = np.zeros(36, dtype=Q8)
        o.or_gelu_mul_quantize_q8_0(fptr(g["geglu_gate"][i]), fptr(g["geglu_up"][i]), 1152, vptr(blocks))
        assert np.array_equal(blocks.view(np.uint8), g["geglu_q8"][i])


def test_l2_prefix_and_pool(g):
    o = oracle()
    for i in range(g["l2_in"].shape[0]):
        v = g["l2_in"][i].copy()
        o.or_l2_normalize(fptr(v), N_EMBD)
        assert np.array_equal(v, g["l2_out"][i])
        for j, dims in enumerate((128, 256, 512, 768)):
            v = g["l2_in"][i].copy()
            assert o.or_normalize_prefix(fptr(v), dims) == 1
            assert np.array_equal(v, g["prefix_out"][i, j])
    out = np.zeros(N_EMBD, np.float32)
    o.or_mean_pool_rms_l2(fptr(g["pool_x"].copy()), g["pool_x"].shape[0], fptr(g["norm_w"]), 1e-6, fptr(out))
    assert np.array_equal(out, g["pool_out"])


@pytest.mark.parametrize("name", ["mm_a", "mm_b"])
def test_q8_gemm(g, name):
    w = q8(g[name + "_w"], g[name + "_w"].shape[0])
    y = gemm_q8_0(w, quantize_q8_0(g[name + "_x"]))
    assert np.array_equal(y, g[name + "_y"])


def test_embedding_rows(g):
    tab = q8(g["embed_table"], 4)
    o = oracle()
    for i in range(4):
        out = np.zeros(N_EMBD, np.float32)
        o.or_dequantize_row_q8_0_scaled(vptr(tab[i]), N_EMBD, np.sqrt(np.float32(768)), fptr(out))
        assert np.array_equal(out, g["embed_out"][i])
    # Dequantisation itself is exact: d * q in fp32 (d has 11 bits, q 8).
    assert np.array_equal(dequantize_q8_0(tab) * np.float32(1.0), dequantize_q8_0(tab))
