"""Per-kernel parity of the gfx950 operators against the CPU oracle, on the
same seeded inputs, through the C ABI (include/eg2_hip.h).

Bit-exact: quantizer, embedding + norm + quantize, residual + norm +
quantize, QK-norm + RoPE (fp16 of the exact fp32 result), pooling, L2 and
Matryoshka prefixes. Tolerance (stated per test): the projection GEMM
(fp16-dequantized operands on MFMA), attention (fp16 operands, fp32
softmax), GeGLU (device tanhf)."""
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


def test_quantize_rows_bit_exact(eg2, gpu):
    import torch

    x = (RNG.standard_normal((96, N_EMBD)) * 10.0 ** RNG.uniform(-5, 3, (96, 1))).astype(np.float32)
    x[0] = 0
    x[1, :32] = 0.5
    x[1, 32:64] = 63.5
    x[2, ::2] = -x[2, ::2]
    q, d = empty((96, N_EMBD), torch.int8, gpu), empty((96, 24), torch.float32, gpu)
    eg2.ops.quantize_rows(dev(x, gpu), q, d)
    wq, wd = split(quantize_q8_0(x), N_EMBD)
    assert np.array_equal(host(q), wq)
    assert np.array_equal(host(d), wd)


def test_embed_norm_quant_bit_exact(eg2, gpu):
    import torch

    vocab = 300
    table = quantize_q8_0((RNG.standard_normal((vocab, N_EMBD)) * 0.05).astype(np.float32))
    ids = RNG.integers(0, vocab, 128).astype(np.int32)
    w = (1 + 0.1 * RNG.standard_normal(N_EMBD)).astype(np.float32)
    scale = float(np.sqrt(np.float32(768)))
    x, xq, xd = empty((128, N_EMBD), torch.float32, gpu), empty((128, N_EMBD), torch.int8, gpu), \
        empty((128, 24), torch.float32, gpu)
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
    assert np.array_equal(host(xq), wq)
    assert np.array_equal(host(xd), wd)


@pytest.mark.parametrize("with_next", [True, False])
def test_residual_norm_quant_bit_exact(eg2, gpu, with_next):
    import torch

    rows = 64
    x = (RNG.standard_normal((rows, N_EMBD)) * 5).astype(np.float32)
    h = (RNG.standard_normal((rows, N_EMBD)) * 0.7).astype(np.float32)
    pw = (1 + 0.1 * RNG.standard_normal(N_EMBD)).astype(np.float32)
    nw = (1 + 0.1 * RNG.standard_normal(N_EMBD)).astype(np.float32)
    xg = dev(x, gpu)
    xq, xd = empty((rows, N_EMBD), torch.int8, gpu), empty((rows, 24), torch.float32, gpu)
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
        assert np.array_equal(host(xq), wq)
        assert np.array_equal(host(xd), wd)


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
    qh, kh, vh = (empty((rows, n), torch.float16, gpu) for n in (N_EMBD, HEAD_DIM, HEAD_DIM))
    eg2.ops.qk_norm_rope(dev(qkv, gpu), dev(qw, gpu), dev(kw, gpu), dev(table, gpu), dev(pos, gpu), 1e-6, qh, kh, vh)
    o = oracle()
    q, k = qkv[:, :N_EMBD].copy(), qkv[:, N_EMBD:N_EMBD + HEAD_DIM].copy()
    for t in range(rows):
        o.or_qk_norm_rope_qk_inplace(fptr(q[t]), fptr(k[t]), fptr(qw), fptr(kw), int(pos[t]), base, 1e-6)
    assert np.array_equal(host(qh).view(np.uint16), q.astype(np.float16).view(np.uint16))
    assert np.array_equal(host(kh).view(np.uint16), k.astype(np.float16).view(np.uint16))
    assert np.array_equal(host(vh).view(np.uint16), qkv[:, N_EMBD + HEAD_DIM:].astype(np.float16).view(np.uint16))


def test_gelu_quant_matches_up_to_tanh_ulps(eg2, gpu):
    """Device tanhf (OCML) and glibc tanhf may differ in the last bit, which
    can move a value across a Q8_0 rounding boundary: every int8 stays within
    1 of the reference and nearly every block is bit-identical."""
    import torch

    rows = 128
    gate = (RNG.standard_normal((rows, N_FF)) * 2).astype(np.float32)
    up = RNG.standard_normal((rows, N_FF)).astype(np.float32)
    gq, gd = empty((rows, N_FF), torch.int8, gpu), empty((rows, 36), torch.float32, gpu)
    eg2.ops.gelu_quant(dev(np.concatenate([gate, up], 1), gpu), gq, gd)
    o = oracle()
    blocks = np.zeros((rows, 36), dtype=Q8)
    for t in range(rows):
        o.or_gelu_mul_quantize_q8_0(fptr(gate[t]), fptr(up[t]), N_FF, vptr(blocks[t]))
    wq, wd = split(blocks, N_FF)
    gq, gd = host(gq), host(gd)
    same_d = gd == wd
    assert same_d.mean() > 0.99
    qd = np.abs(gq.astype(np.int32) - wq).reshape(rows, 36, 32)
    assert qd[same_d].max() <= 1
    assert (qd.max(2) == 0).mean() > 0.98


def _fp16_gemm_double(xq_blocks, w_blocks):
    """The kernel's arithmetic in float64: fp16(q*d) operands, exact sum."""
    a = dequantize_q8_0(xq_blocks).astype(np.float16).astype(np.float64)
    b = dequantize_q8_0(w_blocks).astype(np.float16).astype(np.float64)
    return a @ b.T


@pytest.mark.parametrize("n,m,k", [(512, 2304, 768), (2048, 1280, 768), (33, 40, 64), (16, 3072, 768),
                                   (300, 768, 1152)])
def test_gemm_q8(eg2, gpu, n, m, k):
    """fp32 accumulation of fp16 operands: within 2e-6 relative of the same
    operands summed in float64; within 2e-3 of the scale of the output of the
    reference's exact Q8_0 x Q8_0 dot (fp16 operand rounding, 2^-12)."""
    import torch

    w = quantize_q8_0((RNG.standard_normal((m, k)) * 0.02).astype(np.float32))
    xb = quantize_q8_0(RNG.standard_normal((n, k)).astype(np.float32))
    wq, wd = split(w, k)
    xq, xd = split(xb, k)
    y = empty((n, m), torch.float32, gpu)
    eg2.ops.gemm_q8(dev(xq, gpu), dev(xd, gpu), dev(wq, gpu), dev(wd, gpu), y)
    y = host(y)
    scale = np.abs(y).max()
    assert np.abs(y - _fp16_gemm_double(xb, w)).max() <= 2e-6 * scale
    exact = OL.gemm_q8_0(w, xb)
    assert np.abs(y - exact).max() <= 2e-3 * scale


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


@pytest.mark.parametrize("window", [0, 512])
def test_attention_packed(eg2, gpu, window):
    """Config-2 shape: T=2048 packed from 16 log-uniform segments. The fp16
    MFMA context is compared with the oracle's fp32 context after both go
    through the same Q8_0 quantizer: dequantized values differ by at most one
    quantization step plus 2e-3 of the block scale, and segments never leak."""
    import torch

    rng = np.random.default_rng(2)
    lens = segments_log_uniform(rng)
    T = int(lens.sum())
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint64)
    q = (rng.standard_normal((T, N_EMBD)) * 0.0625).astype(np.float32)
    k = rng.standard_normal((T, HEAD_DIM)).astype(np.float32)
    v = rng.standard_normal((T, HEAD_DIM)).astype(np.float32)
    # Operands are what the device consumes: fp16.
    q, k, v = (a.astype(np.float16).astype(np.float32) for a in (q, k, v))
    lo = np.repeat(offsets[:-1], lens).astype(np.uint32)
    hi = np.repeat(offsets[1:], lens).astype(np.uint32)
    cq, cd = empty((T, N_EMBD), torch.int8, gpu), empty((T, 24), torch.float32, gpu)
    eg2.ops.attention(dev(q.astype(np.float16), gpu), dev(k.astype(np.float16), gpu), dev(v.astype(np.float16), gpu),
                      dev(lo, gpu), dev(hi, gpu), window, cq, cd)
    got = host(cq).astype(np.float32).reshape(T, 24, 32) * host(cd)[:, :, None]
    ctx = np.zeros((T, N_EMBD), np.float32)
    sc = np.zeros(4096, np.float32)
    o = oracle()
    for s in range(len(lens)):
        a, b = int(offsets[s]), int(offsets[s + 1])
        o.or_attention_range(fptr(q[a:b]), fptr(k[a:b]), fptr(v[a:b]), b - a, window, 0, b - a, fptr(ctx[a:b]),
                             fptr(sc))
    step = np.abs(ctx).reshape(T, 24, 32).max(2) / 127.0
    err = np.abs(got - ctx.reshape(T, 24, 32))
    assert (err <= step[:, :, None] * 1.0 + 2e-3 * step[:, :, None] * 127).all()
    ref_blocks = quantize_q8_0(ctx)
    same = (host(cq).reshape(T, 24, 32) == ref_blocks["qs"]).all(2)
    assert same.mean() > 0.5


def test_attention_single_token_segments(eg2, gpu):
    """Length-1 sequences attend only to themselves: the context is v."""
    import torch

    T = 64
    q = RNG.standard_normal((T, N_EMBD)).astype(np.float16)
    k = RNG.standard_normal((T, HEAD_DIM)).astype(np.float16)
    v = RNG.standard_normal((T, HEAD_DIM)).astype(np.float16)
    lo = np.arange(T, dtype=np.uint32)
    cq, cd = empty((T, N_EMBD), torch.int8, gpu), empty((T, 24), torch.float32, gpu)
    eg2.ops.attention(dev(q, gpu), dev(k, gpu), dev(v, gpu), dev(lo, gpu), dev(lo + 1, gpu), 0, cq, cd)
    want = quantize_q8_0(np.tile(v.astype(np.float32), (1, 3)))
    wq, wd = split(want, N_EMBD)
    assert np.array_equal(host(cq), wq)
    assert np.array_equal(host(cd), wd)


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
