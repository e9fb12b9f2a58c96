"""Pins the CPU oracle against mathematics rather than against itself:
closed forms, double-precision brute force, exact-integer known answers,
invariances, and mistakes planted in a brute-force copy that these checks
must reject."""
import numpy as np
import pytest

import oracle_lib as OL
from oracle_lib import N_EMBD, N_FF, HEAD_DIM, Q8, dequantize_q8_0, fptr, gemm_q8_0, oracle, quantize_q8_0, vptr

RNG = np.random.default_rng(7)


def test_fp16_matches_ieee_except_half_up_ties():
    o = oracle()
    x = (RNG.standard_normal(20000) * 10.0 ** RNG.integers(-6, 5, 20000)).astype(np.float32)
    x = x[np.abs(x) < 65504]
    got = np.array([o.or_fp32_to_fp16(float(v)) for v in x], np.uint16)
    rne = x.astype(np.float16).view(np.uint16)
    diff = got != rne
    # Differences are exactly the ties (bits below the kept mantissa = 1000..0),
    # which the reference rounds away from zero in magnitude.
    for v, a, b in zip(x[diff], got[diff], rne[diff]):
        lo = np.float32(np.float16(v))
        hi_bits = int(a)
        assert (hi_bits & 0x7FFF) == (int(b) & 0x7FFF) + 1
        assert abs(float(np.uint16(a).view(np.float16))) > abs(float(lo)) or abs(v) == 0
    # Ties exist in this sample and are resolved upward.
    ties = np.float32([1.0 + 2 ** -11, 2049.0, 0.5 + 2 ** -12])
    for v in ties:
        h = np.uint16(o.or_fp32_to_fp16(float(v))).view(np.float16)
        assert float(h) > float(v)


def test_quantizer_closed_form_properties():
    x = (RNG.standard_normal((400, 32)) * 10.0 ** RNG.uniform(-3, 3, (400, 1))).astype(np.float32)
    x[0] = 0.0
    b = quantize_q8_0(x)[:, 0]
    d = b["d"].view(np.float16).astype(np.float32)
    amax = np.abs(x).max(1)
    # Stored scale is the half-up fp16 of amax/127.
    assert np.array_equal(b["d"], np.array([oracle().or_fp32_to_fp16(float(np.float32(a) / np.float32(127)))
                                            for a in amax], np.uint16))
    q = b["qs"].astype(np.int32)
    assert np.all(q[0] == 0)
    # The largest magnitude maps to +-127 (ties of x*id at 127 cannot exceed it).
    arg = np.abs(x).argmax(1)
    assert np.all(np.abs(q[np.arange(400), arg])[1:] == 127)
    # Each value is within half a step of its quantized value (fp32 step).
    d32 = amax / np.float32(127)
    err = np.abs(x[1:] / d32[1:, None] - q[1:])
    assert err.max() <= 0.5 + 1e-4


def test_quantizer_rounds_half_away_from_zero():
    # amax = 127 * 2^-3 makes d = 2^-3 and id = 8 exact, so x*id is exact.
    x = np.zeros((1, 32), np.float32)
    x[0, 0] = 127 * 0.125
    x[0, 1:5] = np.float32([0.5, -0.5, 1.5, -2.5]) * 0.125
    q = quantize_q8_0(x)[0, 0]["qs"]
    assert list(q[:5]) == [127, 1, -1, 2, -3]


def test_gemm_exact_integer_known_answer():
    # tests/kernels.cpp:61-73 style: operands whose Q8_0 encodings are exact
    # so the projection is integer arithmetic times powers of two.
    n, k, m = 9, 96, 35
    iq = ((np.arange(n * k) % 19) - 9).reshape(n, k).astype(np.int32)
    iq[:, ::32] = 127  # pins amax so d_x = 2^-3 in every block
    x = (iq * 0.125).astype(np.float32)
    wq_i = ((np.arange(m * k) % 23) - 11).reshape(m, k).astype(np.int8)
    w = np.zeros((m, k // 32), dtype=Q8)
    w["d"] = np.float16(0.125).view(np.uint16)
    w["qs"] = wq_i.reshape(m, k // 32, 32)
    y = gemm_q8_0(w, quantize_q8_0(x))
    want = (iq @ wq_i.T.astype(np.int32)).astype(np.float64) * (0.125 * 0.125)
    assert np.array_equal(y.astype(np.float64), want)


def test_gemm_against_double_brute_force():
    n, k, m = 17, 768, 40
    w = quantize_q8_0((RNG.standard_normal((m, k)) * 0.02).astype(np.float32))
    xq = quantize_q8_0(RNG.standard_normal((n, k)).astype(np.float32))
    y = gemm_q8_0(w, xq)
    want = dequantize_q8_0(xq).astype(np.float64) @ dequantize_q8_0(w).astype(np.float64).T
    assert np.abs(y - want).max() <= 1e-6 * np.abs(want).max() + 1e-9


def _softmax_attention_double(q, k, v, window):
    T = q.shape[0]
    out = np.zeros((T, N_EMBD))
    half = window // 2
    for t in range(T):
        lo, hi = (max(t - half, 0), min(t + half + 1, T)) if window > 0 else (0, T)
        for h in range(3):
            s = k[lo:hi].astype(np.float64) @ q[t, h * HEAD_DIM:(h + 1) * HEAD_DIM].astype(np.float64)
            p = np.exp(s - s.max())
            out[t, h * HEAD_DIM:(h + 1) * HEAD_DIM] = (p / p.sum()) @ v[lo:hi].astype(np.float64)
    return out


@pytest.mark.parametrize("T,window", [(1, 0), (19, 0), (40, 0), (40, 10), (40, 512)])
def test_attention_against_double_softmax(T, window):
    q = (RNG.standard_normal((T, N_EMBD)) * 0.2).astype(np.float32)
    k = RNG.standard_normal((T, HEAD_DIM)).astype(np.float32)
    v = RNG.standard_normal((T, HEAD_DIM)).astype(np.float32)
    ctx = np.zeros((T, N_EMBD), np.float32)
    oracle().or_attention_range(fptr(q), fptr(k), fptr(v), T, window, 0, T, fptr(ctx),
                                fptr(np.zeros(4096, np.float32)))
    assert np.abs(ctx - _softmax_attention_double(q, k, v, window)).max() < 2e-5


def test_qk_norm_rope_against_double():
    o = oracle()
    qw = (1 + 0.1 * RNG.standard_normal(256)).astype(np.float32)
    kw = (1 + 0.1 * RNG.standard_normal(256)).astype(np.float32)
    for pos, base in [(0, 1e4), (5, 1e4), (300, 1e6), (2047, 1e4)]:
        q = RNG.standard_normal(N_EMBD).astype(np.float32)
        k = RNG.standard_normal(HEAD_DIM).astype(np.float32)
        qo, ko = q.copy(), k.copy()
        o.or_qk_norm_rope_qk_inplace(fptr(qo), fptr(ko), fptr(qw), fptr(kw), pos, base, 1e-6)
        theta = pos * base ** (-2.0 * np.arange(128) / 256.0)
        c, s = np.cos(theta), np.sin(theta)

        def ref(r, w, scale):
            r = r.astype(np.float64) * w / np.sqrt(np.mean(r.astype(np.float64) ** 2) + 1e-6)
            a, b = r[:128], r[128:]
            return np.concatenate([a * c - b * s, a * s + b * c]) * scale

        want_q = np.concatenate([ref(q[h * 256:(h + 1) * 256], qw, 0.0625) for h in range(3)])
        assert np.abs(qo - want_q).max() < 2e-5
        assert np.abs(ko - ref(k, kw, 1.0)).max() < 2e-4


def test_gelu_against_closed_form():
    x = (RNG.standard_normal(5000) * 5).astype(np.float32)
    got = np.array([oracle().or_gelu_tanh(float(v)) for v in x])
    xd = x.astype(np.float64)
    want = 0.5 * xd * (1 + np.tanh(np.sqrt(2 / np.pi) * (xd + 0.044715 * xd ** 3)))
    assert np.abs(got - want).max() < 5e-6 * max(1.0, np.abs(want).max())


def test_mean_pool_against_double():
    x = (RNG.standard_normal((11, N_EMBD)) * 3).astype(np.float32)
    w = (1 + 0.1 * RNG.standard_normal(N_EMBD)).astype(np.float32)
    out = np.zeros(N_EMBD, np.float32)
    oracle().or_mean_pool_rms_l2(fptr(x.copy()), 11, fptr(w), 1e-6, fptr(out))
    xd = x.astype(np.float64)
    rows = xd * w / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-6)
    want = rows.mean(0)
    want /= np.linalg.norm(want)
    assert np.abs(out - want).max() < 1e-6


# ----------------------------------------------------------- layer composition


def _small_layer(seed, norm_std=0.1):
    rng = np.random.default_rng(seed)

    def mat(m, k):
        return quantize_q8_0((rng.standard_normal((m, k)) * 0.02).astype(np.float32))

    def vec(n):
        return (1 + norm_std * rng.standard_normal(n)).astype(np.float32)

    return dict(attn_q=mat(768, 768), attn_k=mat(256, 768), attn_v=mat(256, 768), attn_output=mat(768, 768),
                ffn_up=mat(1152, 768), ffn_gate=mat(1152, 768), ffn_down=mat(768, 1152), attn_norm=vec(768),
                attn_q_norm=vec(256), attn_k_norm=vec(256), post_attention_norm=vec(768), ffn_norm=vec(768),
                post_ffw_norm=vec(768))


def _layer_double(L, x, offsets, base, window, swap_gate_up=False, skip_post_norm=False):
    """The sandwich layer (EXTRACTION.md:161-169, engine.c:488-821) in float64,
    with the oracle's own Q8_0 quantizer at the reference's quantization points."""
    def rms(v, w):
        return v * w / np.sqrt((v ** 2).mean(-1, keepdims=True) + 1e-6)

    def proj(a, W):
        return dequantize_q8_0(quantize_q8_0(a.astype(np.float32))).astype(np.float64) @ \
            dequantize_q8_0(W).astype(np.float64).T

    x = x.astype(np.float64)
    h = rms(x, L["attn_norm"])
    q, k, v = proj(h, L["attn_q"]), proj(h, L["attn_k"]), proj(h, L["attn_v"])
    pos = np.concatenate([np.arange(offsets[i + 1] - offsets[i]) for i in range(len(offsets) - 1)])
    th = pos[:, None] * base ** (-2.0 * np.arange(128) / 256.0)
    c, s = np.cos(th), np.sin(th)

    def rope(r):
        a, b = r[:, :128], r[:, 128:]
        return np.concatenate([a * c - b * s, a * s + b * c], 1)

    q = np.concatenate([rope(rms(q[:, i * 256:(i + 1) * 256], L["attn_q_norm"])) * 0.0625 for i in range(3)], 1)
    k = rope(rms(k, L["attn_k_norm"]))
    ctx = np.zeros_like(q)
    for sidx in range(len(offsets) - 1):
        a, b = offsets[sidx], offsets[sidx + 1]
        ctx[a:b] = _softmax_attention_double(q[a:b], k[a:b], v[a:b], window)
    o = proj(ctx, L["attn_output"])
    x = x + (o if skip_post_norm else rms(o, L["post_attention_norm"]))
    f = rms(x, L["ffn_norm"])
    up, gate = proj(f, L["ffn_up"]), proj(f, L["ffn_gate"])
    if swap_gate_up:
        up, gate = gate, up
    act = 0.5 * gate * (1 + np.tanh(np.sqrt(2 / np.pi) * (gate + 0.044715 * gate ** 3))) * up
    x = x + rms(proj(act, L["ffn_down"]), L["post_ffw_norm"])
    return x


def _cos(a, b):
    return (a * b).sum(-1) / np.linalg.norm(a, axis=-1) / np.linalg.norm(b, axis=-1)


@pytest.fixture(scope="module")
def layer_case():
    L = _small_layer(11)
    offsets = np.array([0, 5, 13, 14, 33], dtype=np.uint64)
    x = np.random.default_rng(3).standard_normal((33, N_EMBD)).astype(np.float32)
    return L, x, offsets


def test_layer_matches_double_composition(layer_case):
    L, x, offsets = layer_case
    got = OL.layer_forward(L, x, offsets, rope_base=10000.0, window=0, threads=4)
    want = _layer_double(L, x, offsets.astype(np.int64), 10000.0, 0)
    assert _cos(got, want).min() > 0.9999
    assert np.abs(got - want).max() < 0.02


def test_layer_check_rejects_planted_mistakes(layer_case):
    """The composition check above has teeth: plausible mistakes fail it."""
    L, x, offsets = layer_case
    got = OL.layer_forward(L, x, offsets, rope_base=10000.0, window=0, threads=4)
    for kw in (dict(swap_gate_up=True), dict(skip_post_norm=True)):
        bad = _layer_double(L, x, offsets.astype(np.int64), 10000.0, 0, **kw)
        assert np.abs(got - bad).max() > 0.05, kw
    bad_base = _layer_double(L, x, offsets.astype(np.int64), 1e6, 0)
    assert np.abs(got - bad_base).max() > 0.02
    flat = _layer_double(L, x, np.array([0, 33]), 10000.0, 0)  # segments ignored
    assert np.abs(got - flat).max() > 0.05


def test_layer_segments_are_independent(layer_case):
    L, x, offsets = layer_case
    whole = OL.layer_forward(L, x, offsets, threads=4)
    for s in range(len(offsets) - 1):
        a, b = int(offsets[s]), int(offsets[s + 1])
        alone = OL.layer_forward(L, x[a:b], np.array([0, b - a], np.uint64), threads=1)
        assert np.array_equal(alone, whole[a:b])


def test_forward_packing_invariance_and_validation():
    rng = np.random.default_rng(5)
    L = _small_layer(12)
    L.update(rope_base=10000.0, window=0)
    table = np.zeros((OL.VOCAB, 24), dtype=Q8)
    ids = rng.integers(0, OL.VOCAB, 20).astype(np.int32)
    table[np.unique(ids)] = quantize_q8_0((rng.standard_normal((len(np.unique(ids)), 768)) * 0.02).astype(np.float32))
    model = dict(token_embd=table, output_norm=(1 + 0.1 * rng.standard_normal(768)).astype(np.float32),
                 layers=[L, L])
    offsets = np.array([0, 7, 8, 20], np.uint64)
    packed = OL.forward(model, ids, offsets, threads=4)
    for s in range(3):
        a, b = int(offsets[s]), int(offsets[s + 1])
        alone = OL.forward(model, ids[a:b], np.array([0, b - a], np.uint64), threads=1)
        assert np.array_equal(alone[0], packed[s])
    assert np.allclose(np.linalg.norm(packed, axis=1), 1.0, atol=1e-6)
    for bad_ids, bad_off in [(ids, np.array([0, 7, 7, 20])), (ids, np.array([1, 20])),
                             (np.array([-1] + [0] * 19, np.int32), np.array([0, 20]))]:
        with pytest.raises(ValueError):
            OL.forward(model, bad_ids, np.asarray(bad_off, np.uint64))


# ------------------------------------------------------------------ dense head


def _gelu64(g):
    return 0.5 * g * (1 + np.tanh(np.sqrt(2 / np.pi) * (g + 0.044715 * g ** 3)))


def _head_double(rows, offsets, out_w, d2, d3, l2_first=False, requant_mid=True, act=False, transpose_d2=False):
    """EXTRACTION.md:178-181 in float64: per token rms(x, output_norm), the
    mean over the sequence, then dense_2 and dense_3 (no bias), then L2. The
    inputs of both dense projections are Q8_0-quantized with the oracle's
    quantizer (the reference quantizes every projection input, gemma2.c:142-153);
    the keyword arguments plant plausible mistakes."""
    W2 = dequantize_q8_0(d2).astype(np.float64)
    if transpose_d2:  # the [768, 3072] GGUF shape read with its dimensions swapped
        W2 = W2.reshape(N_EMBD, OL.DENSE_FF).T
    W3 = dequantize_q8_0(d3).astype(np.float64)
    out = []
    for s in range(len(offsets) - 1):
        x = rows[offsets[s]:offsets[s + 1]].astype(np.float64)
        r = x * out_w / np.sqrt((x ** 2).mean(1, keepdims=True) + 1e-6)
        p = r.mean(0)
        if l2_first:
            p = p / np.linalg.norm(p)
        pq = dequantize_q8_0(quantize_q8_0(p.astype(np.float32))).astype(np.float64)
        mid = W2 @ pq
        if act:
            mid = _gelu64(mid)
        if requant_mid:
            mid = dequantize_q8_0(quantize_q8_0(mid.astype(np.float32))).astype(np.float64)
        o = W3 @ mid
        out.append(o / np.linalg.norm(o))
    return np.array(out)


def _head_model(seed, norm_scale):
    """A model with no layers (embedding -> pooling -> dense head) whose used
    embedding rows are random."""
    rng = np.random.default_rng(seed)
    lens = [5, 1, 12]
    ids = rng.integers(0, OL.VOCAB, sum(lens)).astype(np.int32)
    table = np.zeros((OL.VOCAB, N_EMBD // 32), dtype=Q8)
    u = np.unique(ids)
    table[u] = quantize_q8_0((rng.standard_normal((len(u), N_EMBD)) * 0.05).astype(np.float32))
    out_w = ((1 + 0.3 * rng.standard_normal(N_EMBD)) * norm_scale).astype(np.float32)
    d2 = quantize_q8_0((rng.standard_normal((OL.DENSE_FF, N_EMBD)) * 0.02).astype(np.float32))
    d3 = quantize_q8_0((rng.standard_normal((N_EMBD, OL.DENSE_FF)) * 0.02).astype(np.float32))
    model = dict(token_embd=table, output_norm=out_w, dense_2=d2, dense_3=d3, layers=[])
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint64)
    rows = dequantize_q8_0(table[ids]) * np.float32(np.sqrt(N_EMBD))
    return model, ids, offsets, rows


@pytest.fixture(scope="module")
def head_cases():
    # norm_scale 1e-5 puts the pooled values' Q8_0 scales in the fp16
    # subnormal range, where normalising first changes the quantized input.
    return {scale: _head_model(17, scale) for scale in (1.0, 1e-5)}


@pytest.mark.parametrize("scale", [1.0, 1e-5])
def test_dense_head_matches_double_composition(head_cases, scale):
    model, ids, offsets, rows = head_cases[scale]
    got = OL.forward(model, ids, offsets, threads=4)
    want = _head_double(rows, offsets.astype(np.int64), model["output_norm"], model["dense_2"], model["dense_3"])
    assert _cos(got, want).min() > 0.999999
    assert np.abs(got - want).max() < 2e-6


def test_dense_head_check_rejects_planted_mistakes(head_cases):
    """The composition check has teeth: each plausible mistake misses its
    tolerance by a wide margin."""
    model, ids, offsets, rows = head_cases[1.0]
    got = OL.forward(model, ids, offsets, threads=4)
    args = (rows, offsets.astype(np.int64), model["output_norm"], model["dense_2"], model["dense_3"])
    for kw in (dict(requant_mid=False), dict(act=True), dict(transpose_d2=True), dict(l2_first=True)):
        bad = _head_double(*args, **kw)
        assert np.abs(got - bad).max() > 1e-4, kw
    # Normalising before the head changes only the quantization of the
    # head's input (Q8_0's fp16 scale rounding is not scale-equivariant);
    # where its block scales fall in the fp16 subnormal range the change is
    # large.
    model, ids, offsets, rows = head_cases[1e-5]
    got = OL.forward(model, ids, offsets, threads=4)
    bad = _head_double(rows, offsets.astype(np.int64), model["output_norm"], model["dense_2"], model["dense_3"],
                       l2_first=True)
    assert np.abs(got - bad).max() > 1e-2


def test_mean_pool_without_l2_is_the_scaled_mean():
    x = (RNG.standard_normal((9, N_EMBD)) * 2).astype(np.float32)
    w = (1 + 0.1 * RNG.standard_normal(N_EMBD)).astype(np.float32)
    mean = np.zeros(N_EMBD, np.float32)
    oracle().or_mean_pool_rms(fptr(x.copy()), 9, fptr(w), 1e-6, fptr(mean))
    xd = x.astype(np.float64)
    want = (xd * w / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-6)).mean(0)
    assert np.abs(mean - want).max() < 1e-6 * np.abs(want).max()
    l2 = np.zeros(N_EMBD, np.float32)
    oracle().or_mean_pool_rms_l2(fptr(x.copy()), 9, fptr(w), 1e-6, fptr(l2))
    m2 = mean.copy()
    oracle().or_l2_normalize(fptr(m2), N_EMBD)
    assert np.array_equal(l2, m2)
