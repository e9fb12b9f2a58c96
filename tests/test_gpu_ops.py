"""Per-kernel parity of the gfx950 operators against the CPU oracle, on the
same seeded inputs, through the C ABI (include/eg2_hip.h).

Bit-exact: quantizer, embedding + norm + quantize, residual + norm +
quantize, QK-norm + RoPE (split fp16 pairs of the exact fp32 result), the
Q8_0 x Q8_0 projection GEMM, pooling, L2 and Matryoshka prefixes.
Tolerance (stated per test): attention (split-fp16 MFMA, fp32 softmax; a
different summation order than the CPU) and GeGLU (GELU through exp2 on the
device, tanhf on the CPU)."""
import numpy as np
import pytest

import oracle_lib as OL
from oracle_lib import N_EMBD, N_FF, HEAD_DIM, Q8, dequantize_q8_0, fptr, oracle, quantize_q8_0, vptr

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(1234)


def dev(a, gpu):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


def empty(shape, dtype, gpu):
    import torch

    return torch.zeros(shape, dtype=dtype, device=gpu)


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def split(blocks, k):
    """Oracle Q8_0 blocks [rows, k/32] -> (int8 [rows, k], float32 scale [rows, k/32])."""
    return blocks["qs"].reshape(blocks.shape[0], k), blocks["d"].view(np.float16).astype(np.float32)


def qbuf(eg2, rows, k, gpu):
    """A device buffer for Q8_0 values of `rows` rows of width k (row tiles)."""
    import torch

    return torch.zeros(eg2.q8_tile_bytes(rows, k), dtype=torch.int8, device=gpu)


def qvals(eg2, t, rows, k):
    """Row-tile Q8_0 values on the device -> int32 [rows, k] on the host."""
    return eg2.q8_unpack_rows(host(t), rows, k).astype(np.int32)


def split_pairs(x):
    """fp32 -> [hi | lo] fp16 rows as the attention operands are stored."""
    hi = x.astype(np.float16)
    lo = (x - hi.astype(np.float32)).astype(np.float16)
    return np.concatenate([hi, lo], axis=-1)


def test_quantize_rows_bit_exact(eg2, gpu):
    import torch

    x = (RNG.standard_normal((96, N_EMBD)) * 10.0 ** RNG.uniform(-5, 3, (96, 1))).astype(np.float32)
    x[0] = 0
    x[1, :32] = 0.5
    x[1, 32:64] = 63.5
    x[2, ::2] = -x[2, ::2]
    q, d = qbuf(eg2, 96, N_EMBD, gpu), empty((24, 96), torch.float32, gpu)
    eg2.ops.quantize_rows(dev(x, gpu), q, d)
    wq, wd = split(quantize_q8_0(x), N_EMBD)
    assert np.array_equal(qvals(eg2, q, 96, N_EMBD), wq)
    assert np.array_equal(host(d).T, wd)


def test_embed_norm_quant_bit_exact(eg2, gpu):
    import torch

    vocab = 300
    table = quantize_q8_0((RNG.standard_normal((vocab, N_EMBD)) * 0.05).astype(np.float32))
    ids = RNG.integers(0, vocab, 128).astype(np.int32)
    w = (1 + 0.1 * RNG.standard_normal(N_EMBD)).astype(np.float32)
    scale = float(np.sqrt(np.float32(768)))
    x, xq, xd = empty((128, N_EMBD), torch.float32, gpu), qbuf(eg2, 128, N_EMBD, gpu), \
        empty((24, 128), torch.float32, gpu)
    eg2.ops.embed_norm_quant(dev(table.view(np.uint8), gpu), dev(ids, gpu), scale, dev(w, gpu), 1e-6, x, xq, xd)
    o = oracle()
    want_x = np.zeros((128, N_EMBD), np.float32)
    for t in range(128):
        o.or_dequantize_row_q8_0_scaled(vptr(table[ids[t]]), N_EMBD, scale, fptr(want_x[t]))
    assert np.array_equal(host(x), want_x)
    blocks = np.zeros((128, 24), dtype=Q8)
    for t in range(128):
        o.or_rms_norm_quantize_q8_0(fptr(want_x[t]), fptr(w), N_EMBD, 1e-6, vptr(blocks[t]))
    wq, wd = split(blocks, N_EMBD)
    assert np.array_equal(qvals(eg2, xq, 128, N_EMBD), wq)
    assert np.array_equal(host(xd).T, wd)


@pytest.mark.parametrize("with_next", [True, False])
def test_residual_norm_quant_bit_exact(eg2, gpu, with_next):
    import torch

    rows = 64
    x = (RNG.standard_normal((rows, N_EMBD)) * 5).astype(np.float32)
    h = (RNG.standard_normal((rows, N_EMBD)) * 0.7).astype(np.float32)
    pw = (1 + 0.1 * RNG.standard_normal(N_EMBD)).astype(np.float32)
    nw = (1 + 0.1 * RNG.standard_normal(N_EMBD)).astype(np.float32)
    xg = dev(x, gpu)
    xq, xd = qbuf(eg2, rows, N_EMBD, gpu), empty((24, rows), torch.float32, gpu)
    eg2.ops.residual_norm_quant(xg, dev(h, gpu), dev(pw, gpu), dev(nw, gpu) if with_next else None, 1e-6, xq, xd)
    o = oracle()
    want = x.copy()
    blocks = np.zeros((rows, 24), dtype=Q8)
    for t in range(rows):
        o.or_rms_norm_residual_inplace(fptr(want[t]), fptr(h[t]), fptr(pw), N_EMBD, 1e-6)
        o.or_rms_norm_quantize_q8_0(fptr(want[t]), fptr(nw), N_EMBD, 1e-6, vptr(blocks[t]))
    assert np.array_equal(host(xg), want)
    if with_next:
        wq, wd = split(blocks, N_EMBD)
        assert np.array_equal(qvals(eg2, xq, rows, N_EMBD), wq)
        assert np.array_equal(host(xd).T, wd)


@pytest.mark.parametrize("base", [10000.0, 1000000.0])
def test_qk_norm_rope_bit_exact(eg2, gpu, base):
    import torch

    rows = 96
    qkv = (RNG.standard_normal((rows, eg2.QKV_COLS)) * 2).astype(np.float32)
    qw = (1 + 0.1 * RNG.standard_normal(HEAD_DIM)).astype(np.float32)
    kw = (1 + 0.1 * RNG.standard_normal(HEAD_DIM)).astype(np.float32)
    pos = RNG.integers(0, 2048, rows).astype(np.int32)
    pos[:3] = [0, 1, 2047]
    table = eg2.rope_table(base)
    qs, ks = (empty((rows, 2 * n), torch.float16, gpu) for n in (N_EMBD, HEAD_DIM))
    # v goes transposed to columns vcol: here two sequences, so the second
    # starts at the next multiple of 32
    vcol, ldv = eg2.attention_vt_columns([0, 40, rows])
    vt = empty((2, HEAD_DIM, ldv), torch.float16, gpu)
    eg2.ops.qk_norm_rope(dev(qkv, gpu), dev(qw, gpu), dev(kw, gpu), dev(table, gpu), dev(pos, gpu), dev(vcol, gpu),
                         1e-6, qs, ks, vt)
    assert vcol[39] == 39 and vcol[40] == 64
    vt = host(vt)
    assert not vt[:, :, 40:64].any()  # columns between the sequences stay untouched
    vs = torch.from_numpy(np.concatenate([vt[0][:, vcol].T, vt[1][:, vcol].T], axis=1))
    o = oracle()
    q, k = qkv[:, :N_EMBD].copy(), qkv[:, N_EMBD:N_EMBD + HEAD_DIM].copy()
    for t in range(rows):
        o.or_qk_norm_rope_qk_inplace(fptr(q[t]), fptr(k[t]), fptr(qw), fptr(kw), int(pos[t]), base, 1e-6)
    v = qkv[:, N_EMBD + HEAD_DIM:]
    for got, want in ((qs, q * np.float32(16)), (ks, k), (vs, v)):
        got = host(got) if got.is_cuda else got.numpy()
        assert np.array_equal(got.view(np.uint16), split_pairs(want).view(np.uint16))
        # hi + lo recovers the fp32 value to 22 significand bits.
        w = got.shape[1] // 2
        rec = got[:, :w].astype(np.float64) + got[:, w:].astype(np.float64)
        assert np.abs(rec - want).max() <= 2.0 ** -21 * np.abs(want).max()


def test_gelu_quant_matches_up_to_tanh_ulps(eg2, gpu):
    """The device GELU (g / (1 + e^(-2z))) and the CPU's 0.5 g (1 + tanhf(z))
    differ in the last bits, which can move a value across a Q8_0 rounding
    boundary: every int8 stays within 1 of the reference and nearly every
    block is bit-identical."""
    import torch

    rows = 128
    gate = (RNG.standard_normal((rows, N_FF)) * 2).astype(np.float32)
    up = RNG.standard_normal((rows, N_FF)).astype(np.float32)
    gq, gd = qbuf(eg2, rows, N_FF, gpu), empty((36, rows), torch.float32, gpu)
    eg2.ops.gelu_quant(dev(np.concatenate([gate, up], 1), gpu), gq, gd)
    o = oracle()
    blocks = np.zeros((rows, 36), dtype=Q8)
    for t in range(rows):
        o.or_gelu_mul_quantize_q8_0(fptr(gate[t]), fptr(up[t]), N_FF, vptr(blocks[t]))
    wq, wd = split(blocks, N_FF)
    gq, gd = qvals(eg2, gq, rows, N_FF), host(gd).T
    same_d = gd == wd
    assert same_d.mean() > 0.99
    qd = np.abs(gq.astype(np.int32) - wq).reshape(rows, 36, 32)
    assert qd[same_d].max() <= 1
    assert (qd.max(2) == 0).mean() > 0.98


def device_q8(eg2, blocks, k, gpu):
    """Oracle Q8_0 activation blocks -> the kernels' layout (int8 row tiles
    + float scales transposed [k/32, rows])."""
    q, d = split(blocks, k)
    return dev(eg2.q8_pack_rows(q), gpu), dev(d.T, gpu)


def device_weights(eg2, blocks, k, gpu):
    """Oracle Q8_0 weight blocks -> the GEMM's weight operands."""
    wq, wd = eg2.q8_weight_tiles(blocks.view(np.uint8), blocks.shape[0], k)
    return dev(wq, gpu), dev(wd, gpu)


@pytest.mark.parametrize("n,m,k", [(512, 2304, 768), (2048, 1280, 768), (2048, 768, 1152), (33, 40, 64),
                                   (16, 3072, 768), (16, 768, 3072), (300, 768, 1152), (1, 32, 32)])
def test_gemm_q8_bit_exact(eg2, gpu, n, m, k):
    """Config 1 (512 x 2304 x 768) and every projection shape of the forward:
    identical to the reference's Q8_0 x Q8_0 dot (gemma2.c:120-141)."""
    import torch

    w = quantize_q8_0((RNG.standard_normal((m, k)) * 0.02).astype(np.float32))
    xb = quantize_q8_0(RNG.standard_normal((n, k)).astype(np.float32))
    xb[0, 0]["qs"][:] = -128  # the most negative Q8_0 value round-trips too
    y = empty((n, m), torch.float32, gpu)
    eg2.ops.gemm_q8(*device_q8(eg2, xb, k, gpu), *device_weights(eg2, w, k, gpu), y)
    assert np.array_equal(host(y), OL.gemm_q8_0(w, xb))


def test_gemm_q8_strided_output(eg2, gpu):
    """ldy > m writes into a wider row (the fused-projection layout)."""
    import torch

    n, m, k = 64, 96, 768
    w = quantize_q8_0((RNG.standard_normal((m, k)) * 0.02).astype(np.float32))
    xb = quantize_q8_0(RNG.standard_normal((n, k)).astype(np.float32))
    y = torch.full((n, 160), 7.0, dtype=torch.float32, device=gpu)
    eg2.ops.gemm_q8(*device_q8(eg2, xb, k, gpu), *device_weights(eg2, w, k, gpu), y, m=m)
    got = host(y)
    assert np.array_equal(got[:, :m], OL.gemm_q8_0(w, xb))
    assert (got[:, m:] == 7.0).all()


def run_geglu(eg2, gpu, xb, wg, wu, k, ff, ldg):
    """The fused gate|up + GeGLU GEMM on oracle Q8_0 blocks; returns
    (int8 values [n, ff], scales [ff/32, ldg]) with sentinels left in the
    unwritten scale columns."""
    import torch

    n = xb.shape[0]
    wq, wd = eg2.q8_geglu_weight_tiles(wg.view(np.uint8), wu.view(np.uint8), ff, k)
    gq = qbuf(eg2, n, ff, gpu)
    gd = torch.full((ff // 32, ldg), -3.0, dtype=torch.float32, device=gpu)
    eg2.ops.gemm_q8_geglu(*device_q8(eg2, xb, k, gpu), dev(wq, gpu), dev(wd, gpu), gq, gd, n)
    return qvals(eg2, gq, n, ff), host(gd)


@pytest.mark.parametrize("n", [2048, 300, 33, 1])
def test_gemm_q8_geglu_equals_gemm_then_gelu_quant(eg2, gpu, n):
    """The fused kernel of the forward (gate|up 2304 x 768 + GeGLU + Q8_0)
    is bit-identical to the two-kernel path: eg2_hip_gemm_q8 on
    [gate | up], then eg2_hip_gelu_quant."""
    import torch

    k, ff = N_EMBD, N_FF
    wg = quantize_q8_0((RNG.standard_normal((ff, k)) * 0.02).astype(np.float32))
    wu = quantize_q8_0((RNG.standard_normal((ff, k)) * 0.02).astype(np.float32))
    xb = quantize_q8_0(RNG.standard_normal((n, k)).astype(np.float32))
    q, d = run_geglu(eg2, gpu, xb, wg, wu, k, ff, n + 5)
    y = empty((n, 2 * ff), torch.float32, gpu)
    eg2.ops.gemm_q8(*device_q8(eg2, xb, k, gpu), *device_weights(eg2, np.concatenate([wg, wu]), k, gpu), y)
    rq, rd = qbuf(eg2, n, ff, gpu), empty((36, n), torch.float32, gpu)
    eg2.ops.gelu_quant(y, rq, rd)
    assert np.array_equal(q, qvals(eg2, rq, n, ff))
    assert np.array_equal(d[:, :n], host(rd))
    assert (d[:, n:] == -3.0).all()


@pytest.mark.parametrize("n,ff,k", [(64, 32, 32), (100, 96, 160), (65, 1152, 768)])
def test_gemm_q8_geglu_against_oracle(eg2, gpu, n, ff, k):
    """Other widths (k = 160: a block count that is not a multiple of the
    LDS ring depth) against the oracle: the GEMM is exact, so only the
    GELU's last bits separate the results (the tolerance of
    test_gelu_quant_matches_up_to_tanh_ulps)."""
    wg = quantize_q8_0((RNG.standard_normal((ff, k)) * 0.05).astype(np.float32))
    wu = quantize_q8_0((RNG.standard_normal((ff, k)) * 0.05).astype(np.float32))
    xb = quantize_q8_0(RNG.standard_normal((n, k)).astype(np.float32))
    q, d = run_geglu(eg2, gpu, xb, wg, wu, k, ff, n)
    gate, up = OL.gemm_q8_0(wg, xb), OL.gemm_q8_0(wu, xb)
    o = oracle()
    nb = ff // 32
    blocks = np.zeros((n, nb), dtype=Q8)
    for t in range(n):
        o.or_gelu_mul_quantize_q8_0(fptr(np.ascontiguousarray(gate[t])), fptr(np.ascontiguousarray(up[t])), ff,
                                    vptr(blocks[t]))
    wq, wd = split(blocks, ff)
    same_d = d.T == wd
    assert same_d.mean() > 0.99
    qd = np.abs(q - wq).reshape(n, nb, 32)
    assert qd[same_d].max() <= 1
    assert (qd.max(2) == 0).mean() > 0.98


@pytest.mark.parametrize("lens", [[128] * 16, [40, 260], [33], [1, 1, 5], [2048]])
def test_gemm_q8_qkv_rope_equals_gemm_then_qk_norm_rope(eg2, gpu, lens):
    """The fused QKV projection + QK-norm/RoPE of the forward is
    bit-identical to eg2_hip_gemm_q8 on [q|k|v] then eg2_hip_qk_norm_rope:
    q and k split pairs, and v transposed at each token's column (columns
    no token writes stay untouched)."""
    import torch

    k = N_EMBD
    n = int(sum(lens))
    offsets = np.concatenate([[0], np.cumsum(lens)])
    w = quantize_q8_0((RNG.standard_normal((eg2.QKV_COLS, k)) * 0.05).astype(np.float32))
    xb = quantize_q8_0(RNG.standard_normal((n, k)).astype(np.float32))
    xq, xd = device_q8(eg2, xb, k, gpu)
    wq, wd = device_weights(eg2, w, k, gpu)
    qw, kw = ((1 + 0.1 * RNG.standard_normal(HEAD_DIM)).astype(np.float32) for _ in range(2))
    pos = np.concatenate([np.arange(l) for l in lens]).astype(np.int32)
    table = dev(eg2.rope_table(1e4), gpu)
    vcol, ldv = eg2.attention_vt_columns(offsets)
    args = (dev(qw, gpu), dev(kw, gpu), table, dev(pos, gpu), dev(vcol, gpu), 1e-6)
    outs = []
    for fused in (False, True):
        qs, ks = (torch.full((n, 2 * c), 7.0, dtype=torch.float16, device=gpu) for c in (N_EMBD, HEAD_DIM))
        vt = torch.full((2, HEAD_DIM, ldv), 7.0, dtype=torch.float16, device=gpu)
        if fused:
            eg2.ops.gemm_q8_qkv_rope(xq, xd, wq, wd, n, *args, qs, ks, vt)
        else:
            y = empty((n, eg2.QKV_COLS), torch.float32, gpu)
            eg2.ops.gemm_q8(xq, xd, wq, wd, y)
            eg2.ops.qk_norm_rope(y, *args, qs, ks, vt)
        outs.append([host(t).view(np.uint16) for t in (qs, ks, vt)])
    for a, b in zip(*outs):
        assert np.array_equal(a, b)


def segments_log_uniform(rng, n_seg=16, total=2048, lo=8, hi=512):
    """Sequence lengths ~ exp(U(ln lo, ln hi)), scaled to sum `total`,
    rounded, each clipped to [lo, hi]; the remainder goes to the last one
    (clipped as well, any leftover is spread over the others)."""
    raw = np.exp(rng.uniform(np.log(lo), np.log(hi), n_seg))
    lens = np.clip(np.round(raw / raw.sum() * total).astype(np.int64), lo, hi)
    lens[-1] = np.clip(total - lens[:-1].sum(), lo, hi)
    i = 0
    while lens.sum() != total:
        step = 1 if lens.sum() < total else -1
        if lo <= lens[i % (n_seg - 1)] + step <= hi:
            lens[i % (n_seg - 1)] += step
        i += 1
    return lens


def transposed_v(eg2, v, offsets, gpu, fill=0.0):
    """v [T, 256] -> (vt [2, 256, ldv] split fp16 at the columns of
    eg2_attention_vt_columns, vcol); other columns hold `fill`."""
    vcol, ldv = eg2.attention_vt_columns(offsets)
    vt = np.full((2, HEAD_DIM, ldv), fill, dtype=np.float16)
    pairs = split_pairs(v)
    vt[0][:, vcol] = pairs[:, :HEAD_DIM].T
    vt[1][:, vcol] = pairs[:, HEAD_DIM:].T
    return dev(vt, gpu), dev(vcol, gpu)


def run_attention(eg2, gpu, q, k, v, offsets, window, fill=0.0):
    import torch

    T = q.shape[0]
    cq, cd = qbuf(eg2, T, N_EMBD, gpu), empty((24, T), torch.float32, gpu)
    vt, _ = transposed_v(eg2, v, offsets, gpu, fill)
    eg2.ops.attention(dev(split_pairs(q * np.float32(16)), gpu), dev(split_pairs(k), gpu), vt, offsets, window, cq,
                      cd)
    return qvals(eg2, cq, T, N_EMBD), np.ascontiguousarray(host(cd).T)


def attention_double(q, k, v, offsets, window):
    """Exact (float64) softmax attention per sequence, 3 query heads sharing one KV head."""
    T = q.shape[0]
    out = np.zeros((T, N_EMBD))
    half = window // 2
    for s in range(len(offsets) - 1):
        a, b = int(offsets[s]), int(offsets[s + 1])
        kk, vv = k[a:b].astype(np.float64), v[a:b].astype(np.float64)
        for h in range(3):
            sc = q[a:b, h * 256:(h + 1) * 256].astype(np.float64) @ kk.T
            if window > 0:
                i = np.arange(b - a)
                sc[np.abs(i[:, None] - i[None, :]) > half] = -np.inf
            p = np.exp(sc - sc.max(1, keepdims=True))
            out[a:b, h * 256:(h + 1) * 256] = (p / p.sum(1, keepdims=True)) @ vv
    return out


@pytest.mark.parametrize("window", [0, 512])
def test_attention_packed(eg2, gpu, window):
    """Config-2 shape: T=2048 packed from 16 log-uniform segments (8..512).
    Q8_0 quantizes with the fp32 step d = amax/127 but stores d rounded to
    fp16 (quants.c:128-134), so a dequantized value lies within
    (0.5 + 127 * 2^-11) * d of its input. Against float64 attention, every
    dequantized device value meets that bound (with the stored scale, 2^-10
    slack) plus 2^-16 * max|v|, an fp32-level accumulation error over up to
    512 keys; the oracle's fp32 context is within the same 2^-16 * max|v|.
    After the shared quantizer more than 99.5% of blocks are identical to the
    oracle's; the others sit on rounding boundaries where the two fp32
    summation orders (the CPU's sequential sum and the MFMA's) round apart."""
    rng = np.random.default_rng(2)
    lens = segments_log_uniform(rng)
    T = int(lens.sum())
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint64)
    q = (rng.standard_normal((T, N_EMBD)) * 0.0625).astype(np.float32)
    k = rng.standard_normal((T, HEAD_DIM)).astype(np.float32)
    v = rng.standard_normal((T, HEAD_DIM)).astype(np.float32)
    cq, cd = run_attention(eg2, gpu, q, k, v, offsets, window)
    ctx = np.zeros((T, N_EMBD), np.float32)
    sc = np.zeros(4096, np.float32)
    o = oracle()
    for s in range(len(lens)):
        a, b = int(offsets[s]), int(offsets[s + 1])
        o.or_attention_range(fptr(q[a:b]), fptr(k[a:b]), fptr(v[a:b]), b - a, window, 0, b - a, fptr(ctx[a:b]),
                             fptr(sc))
    exact = attention_double(q, k, v, offsets, window)
    tol = 2.0 ** -16 * np.abs(v).max()
    assert np.abs(ctx - exact).max() <= tol
    got = cq.astype(np.float32).reshape(T, 24, 32) * cd[:, :, None]
    err = np.abs(got - exact.reshape(T, 24, 32))
    bound = (0.5 + 127 * 2.0 ** -11) * (1 + 2.0 ** -10) * cd[:, :, None] + tol
    print(f"max (error - tol) / step: {((err - tol) / cd[:, :, None]).max():.5f}")
    assert (err <= bound).all()
    ref = quantize_q8_0(ctx)
    same = (cq.reshape(T, 24, 32) == ref["qs"]).all(2) & (cd == ref["d"].view(np.float16).astype(np.float32))
    print(f"identical Q8_0 blocks vs the oracle: {same.mean():.5f}")
    assert same.mean() > 0.995


@pytest.mark.parametrize("lens", [[1100, 600, 300, 48], [2048]])
def test_attention_long_sequences_split(eg2, gpu, lens):
    """Sequences longer than 256 tokens run as 256-key chunks whose partial
    softmax results are merged: the same float64 bound as the unsplit
    path, the same agreement with the oracle's quantized context, and a
    split sequence gives the same bits alone as packed."""
    rng = np.random.default_rng(sum(lens))
    T = sum(lens)
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint64)
    q = (rng.standard_normal((T, N_EMBD)) * 0.0625).astype(np.float32)
    k = rng.standard_normal((T, HEAD_DIM)).astype(np.float32)
    v = rng.standard_normal((T, HEAD_DIM)).astype(np.float32)
    cq, cd = run_attention(eg2, gpu, q, k, v, offsets, 0)
    exact = attention_double(q, k, v, offsets, 0)
    tol = 2.0 ** -16 * np.abs(v).max()
    got = cq.astype(np.float32).reshape(T, 24, 32) * cd[:, :, None]
    bound = (0.5 + 127 * 2.0 ** -11) * (1 + 2.0 ** -10) * cd[:, :, None] + tol
    assert (np.abs(got - exact.reshape(T, 24, 32)) <= bound).all()
    ctx = np.zeros((T, N_EMBD), np.float32)
    sc = np.zeros(4096, np.float32)
    for s in range(len(lens)):
        a, b = int(offsets[s]), int(offsets[s + 1])
        oracle().or_attention_range(fptr(q[a:b]), fptr(k[a:b]), fptr(v[a:b]), b - a, 0, 0, b - a, fptr(ctx[a:b]),
                                    fptr(sc))
    ref = quantize_q8_0(ctx)
    same = (cq.reshape(T, 24, 32) == ref["qs"]).all(2) & (cd == ref["d"].view(np.float16).astype(np.float32))
    print(f"identical Q8_0 blocks vs the oracle: {same.mean():.5f}")
    assert same.mean() > 0.995
    if len(lens) > 1:
        a, b = int(offsets[1]), int(offsets[2])
        sq, sd = run_attention(eg2, gpu, q[a:b], k[a:b], v[a:b], [0, b - a], 0)
        assert np.array_equal(sq, cq[a:b]) and np.array_equal(sd, cd[a:b])


def test_attention_single_token_segments(eg2, gpu):
    """Length-1 sequences attend only to themselves: the context is v
    (to the 22 bits of the split operands), quantized like the reference."""
    T = 64
    q = RNG.standard_normal((T, N_EMBD)).astype(np.float32)
    k = RNG.standard_normal((T, HEAD_DIM)).astype(np.float32)
    v = RNG.standard_normal((T, HEAD_DIM)).astype(np.float32)
    cq, cd = run_attention(eg2, gpu, q, k, v, np.arange(T + 1), 0)
    wq, wd = split(quantize_q8_0(np.tile(v, (1, 3))), N_EMBD)
    assert (cd == wd).mean() > 0.999
    assert np.abs(cq - wq).max() <= 1
    assert (cq == wq).mean() > 0.999


@pytest.mark.parametrize("window", [0, 16])
def test_attention_independent_of_packing(eg2, gpu, window):
    """A sequence gives bit-identical context alone or anywhere in a wave."""
    rng = np.random.default_rng(8)
    lens = [37, 5, 64, 1, 100, 33]
    T = sum(lens)
    offsets = np.concatenate([[0], np.cumsum(lens)])
    q = (rng.standard_normal((T, N_EMBD)) * 0.0625).astype(np.float32)
    k = rng.standard_normal((T, HEAD_DIM)).astype(np.float32)
    v = rng.standard_normal((T, HEAD_DIM)).astype(np.float32)
    cq, cd = run_attention(eg2, gpu, q, k, v, offsets, window)
    for s in range(len(lens)):
        a, b = offsets[s], offsets[s + 1]
        sq, sd = run_attention(eg2, gpu, q[a:b], k[a:b], v[a:b], [0, b - a], window)
        assert np.array_equal(sq, cq[a:b]) and np.array_equal(sd, cd[a:b])


def test_attention_ignores_unused_vt_columns(eg2, gpu):
    """Key tiles overrun short sequences into their 32-aligned column
    padding; those keys are masked, so any finite filler gives the same bits."""
    rng = np.random.default_rng(9)
    lens = [3, 40, 1, 70]
    T = sum(lens)
    offsets = np.concatenate([[0], np.cumsum(lens)])
    q = (rng.standard_normal((T, N_EMBD)) * 0.0625).astype(np.float32)
    k = rng.standard_normal((T, HEAD_DIM)).astype(np.float32)
    v = rng.standard_normal((T, HEAD_DIM)).astype(np.float32)
    a = run_attention(eg2, gpu, q, k, v, offsets, 0, fill=0.0)
    b = run_attention(eg2, gpu, q, k, v, offsets, 0, fill=1000.0)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_pool_and_l2_bit_exact(eg2, gpu):
    import torch

    lens = [1, 7, 130, 2, 60]
    T = sum(lens)
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
    x = (RNG.standard_normal((T, N_EMBD)) * 4).astype(np.float32)
    w = (1 + 0.1 * RNG.standard_normal(N_EMBD)).astype(np.float32)
    xg = dev(x, gpu)
    eg2.ops.rms_norm_rows(xg, dev(w, gpu), 1e-6)
    out = empty((len(lens), N_EMBD), torch.float32, gpu)
    eg2.ops.pool_l2(xg, dev(offsets, gpu), out)
    o = oracle()
    want = np.zeros((len(lens), N_EMBD), np.float32)
    for s in range(len(lens)):
        a, b = offsets[s], offsets[s + 1]
        o.or_mean_pool_rms_l2(fptr(x[a:b].copy()), int(b - a), fptr(w), 1e-6, fptr(want[s]))
    assert np.array_equal(host(out), want)


@pytest.mark.parametrize("lens", [[2048], [1, 700, 300, 1047], [257, 5, 33], [1]])
def test_pool_mean_then_l2_equals_pool_l2(eg2, gpu, lens):
    """The column-split mean (12 workgroups per sequence, the executor's
    form for waves with a sequence over 256 tokens) followed by the
    full-width L2 is eg2_hip_pool_l2 bit for bit, and both match the
    oracle's mean + L2."""
    import torch

    T = sum(lens)
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
    x = (RNG.standard_normal((T, N_EMBD)) * 4).astype(np.float32)
    xg, og = dev(x, gpu), dev(offsets, gpu)
    one = empty((len(lens), N_EMBD), torch.float32, gpu)
    eg2.ops.pool_l2(xg, og, one)
    two = empty((len(lens), N_EMBD), torch.float32, gpu)
    eg2.ops.pool_mean(xg, og, two)
    mean = host(two).copy()
    eg2.ops.l2_prefix(two, N_EMBD)
    assert np.array_equal(host(one), host(two))
    # the mean half alone: token-order float32 sums scaled by 1/n
    for s in range(len(lens)):
        a, b = offsets[s], offsets[s + 1]
        acc = np.zeros(N_EMBD, np.float32)
        for t in range(a, b):
            acc = (acc + x[t]).astype(np.float32)
        assert np.array_equal(mean[s], (acc * (np.float32(1) / np.float32(b - a))).astype(np.float32))


@pytest.mark.parametrize("dims", [128, 256, 512, 768])
def test_l2_prefix_bit_exact(eg2, gpu, dims):
    e = RNG.standard_normal((20, N_EMBD)).astype(np.float32)
    eg = dev(e, gpu)
    eg2.ops.l2_prefix(eg, dims)
    want = e.copy()
    for i in range(20):
        assert oracle().or_normalize_prefix(fptr(want[i]), dims) == 1 or dims == 768
        if dims == 768:
            oracle().or_l2_normalize(fptr(want[i]), 768)
    assert np.array_equal(host(eg), want)
