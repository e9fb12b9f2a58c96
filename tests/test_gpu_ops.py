"""Per-kernel parity of the gfx950 operators against the CPU oracle, on the
same seeded inputs, through the C ABI (include/eg2_hip.h).

Every kernel is bit-exact: quantizer, embedding + norm + quantize, residual +
norm + quantize, QK-norm + RoPE, GeGLU (+ its Q8_0; the host libm's tanhf
restated on the device), the Q8_0 x Q8_0 projection GEMM and its fused
forms, attention (the reference's dot order, expf and summation order) with
the Q8_0 of its context, pooling, L2 and Matryoshka prefixes; and the
device's expf / tanhf equal the host libm's over a sweep of all floats."""
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


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


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


@pytest.mark.parametrize("with_next,rows", [(True, 64), (False, 64), (True, 37), (False, 5)])
def test_residual_norm_quant_bit_exact(eg2, gpu, with_next, rows):
    """Rows go 8 to a workgroup; 37 and 5 leave a partial last group."""
    import torch

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


def test_residual_norm_quant_zero_and_subnormal_blocks(eg2, gpu):
    """The next norm's weight zero over block 0 and subnormal over block 1 of
    every row: an all-zero block (1/d = 0, every value quantizes to 0) and a
    block whose 1/d overflows (every value -128, as the reference's
    conversion gives), each from the lane that computes its group's scale and
    broadcast to the group; the other blocks as usual. Bit for bit the
    oracle's."""
    import torch

    rows = 48
    x = (RNG.standard_normal((rows, N_EMBD)) * 5).astype(np.float32)
    h = (RNG.standard_normal((rows, N_EMBD)) * 0.7).astype(np.float32)
    pw = (1 + 0.1 * RNG.standard_normal(N_EMBD)).astype(np.float32)
    nw = (1 + 0.1 * RNG.standard_normal(N_EMBD)).astype(np.float32)
    nw[:32] = 0.0
    nw[32:64] = np.float32(1e-41)
    xg = dev(x, gpu)
    xq, xd = qbuf(eg2, rows, N_EMBD, gpu), empty((24, rows), torch.float32, gpu)
    eg2.ops.residual_norm_quant(xg, dev(h, gpu), dev(pw, gpu), dev(nw, gpu), 1e-6, xq, xd)
    o = oracle()
    want = x.copy()
    blocks = np.zeros((rows, 24), dtype=Q8)
    for t in range(rows):
        o.or_rms_norm_residual_inplace(fptr(want[t]), fptr(h[t]), fptr(pw), N_EMBD, 1e-6)
        o.or_rms_norm_quantize_q8_0(fptr(want[t]), fptr(nw), N_EMBD, 1e-6, vptr(blocks[t]))
    wq, wd = split(blocks, N_EMBD)
    assert (wq[:, :32] == 0).all() and (wq[:, 32:64] == -128).all()  # the two cases do occur
    assert np.array_equal(host(xg), want)
    assert np.array_equal(qvals(eg2, xq, rows, N_EMBD), wq)
    assert np.array_equal(bits(host(xd).T), bits(wd))


def oracle_qk_norm_rope(qkv, qw, kw, pos, base):
    q, k = qkv[:, :N_EMBD].copy(), qkv[:, N_EMBD:N_EMBD + HEAD_DIM].copy()
    o = oracle()
    for t in range(qkv.shape[0]):
        o.or_qk_norm_rope_qk_inplace(fptr(q[t]), fptr(k[t]), fptr(qw), fptr(kw), int(pos[t]), base, 1e-6)
    return np.concatenate([q, k, qkv[:, N_EMBD + HEAD_DIM:]], axis=1)


@pytest.mark.parametrize("base", [10000.0, 1000000.0])
def test_qk_norm_rope_bit_exact(eg2, gpu, base):
    """Rows [q0 q1 q2 | k | v]: q and k normalised and rotated bit for bit
    like the oracle, v unchanged; the same in place."""
    import torch

    rows = 96
    qkv = (RNG.standard_normal((rows, eg2.QKV_COLS)) * 2).astype(np.float32)
    qw = (1 + 0.1 * RNG.standard_normal(HEAD_DIM)).astype(np.float32)
    kw = (1 + 0.1 * RNG.standard_normal(HEAD_DIM)).astype(np.float32)
    pos = RNG.integers(0, 2048, rows).astype(np.int32)
    pos[:3] = [0, 1, 2047]
    table = dev(eg2.rope_table(base), gpu)
    want = oracle_qk_norm_rope(qkv, qw, kw, pos, base)
    out = torch.full((rows, eg2.QKV_COLS), 7.0, device=gpu)
    x = dev(qkv, gpu)
    eg2.ops.qk_norm_rope(x, dev(qw, gpu), dev(kw, gpu), table, dev(pos, gpu), 1e-6, out)
    assert np.array_equal(bits(host(out)), bits(want))
    eg2.ops.qk_norm_rope(x, dev(qw, gpu), dev(kw, gpu), table, dev(pos, gpu), 1e-6, x)
    assert np.array_equal(bits(host(x)), bits(want))


def oracle_gelu_q8(gate, up):
    o = oracle()
    blocks = np.zeros((gate.shape[0], gate.shape[1] // 32), dtype=Q8)
    for t in range(gate.shape[0]):
        o.or_gelu_mul_quantize_q8_0(fptr(np.ascontiguousarray(gate[t])), fptr(np.ascontiguousarray(up[t])),
                                    gate.shape[1], vptr(blocks[t]))
    return split(blocks, gate.shape[1])


def test_gelu_quant_bit_exact(eg2, gpu):
    """gelu_tanh(gate) * up and its Q8_0, with the host libm's tanhf restated
    on the device: bit for bit the oracle's, over gates spanning every
    branch of tanhf / expm1f (|z| tiny, < 1, >= 1, >= 22)."""
    import torch

    rows = 128
    gate = (RNG.standard_normal((rows, N_FF)) * 2).astype(np.float32)
    gate[0, :64] = np.float32([0.0, -0.0, 1e-30, -1e-30, 1e-10, 3e-8, 0.5, -0.5, 1.0, -1.0, 1.2, -1.2, 5.0, -5.0,
                               9.0, -9.0, 12.0, -12.0, 30.0, -30.0, 100.0, -100.0, 1e-3, -1e-3] + [2.0] * 40)
    gate[1] = np.linspace(-40, 40, N_FF, dtype=np.float32)
    up = RNG.standard_normal((rows, N_FF)).astype(np.float32)
    gq, gd = qbuf(eg2, rows, N_FF, gpu), empty((36, rows), torch.float32, gpu)
    eg2.ops.gelu_quant(dev(np.concatenate([gate, up], 1), gpu), gq, gd)
    wq, wd = oracle_gelu_q8(gate, up)
    assert np.array_equal(qvals(eg2, gq, rows, N_FF), wq)
    assert np.array_equal(bits(host(gd).T), bits(wd))


def test_tanh_approximation_error_bound(eg2, gpu):
    """The GeGLU kernels certify each Q8_0 result from an approximate tanh
    whose distance to the host tanhf (as restated) they take to be at most
    2^-21: checked over every finite float on the device."""
    import torch

    out = torch.zeros(1, dtype=torch.int32, device=gpu)
    eg2.check(eg2.lib().eg2_hip_tanh_approx_error(eg2.ops._p(out), eg2.ops._stream()), "tanh_approx_error")
    worst = host(out).view(np.float32)[0]
    print(f"max |tanh_approx - tanhf| = {worst!r} ({worst * 2.0 ** 24:.2f} units of 2^-24)")
    assert 0 < worst <= 2.0 ** -21


def test_gelu_quant_certified_against_oracle(eg2, gpu):
    """The GeGLU quantization decides most values from the approximation and
    its bound, and evaluates the exact tanhf for the block maxima and the
    values whose interval straddles a rounding boundary: bit for bit the
    oracle's on 4096 x 1152 values of several distributions (about 2,000
    straddling values at the measured rate of 1 in 2,000), plus blocks of
    equal values (every value a candidate maximum), two tied maxima, zeros,
    subnormals, huge gates (tanh = +-1) and strongly negative gates (the
    bound dominated by |g u|)."""
    import torch

    rng = np.random.default_rng(77)
    rows = 4096
    gate = np.empty((rows, N_FF), np.float32)
    up = np.empty((rows, N_FF), np.float32)
    q = rows // 4
    gate[:q] = rng.standard_normal((q, N_FF)) * 2
    up[:q] = rng.standard_normal((q, N_FF))
    gate[q:2 * q] = rng.standard_normal((q, N_FF)) * 0.3
    up[q:2 * q] = rng.standard_normal((q, N_FF)) * 5
    gate[2 * q:3 * q] = -np.abs(rng.standard_normal((q, N_FF)) * 4)  # tiny 1 + tanh
    up[2 * q:3 * q] = rng.standard_normal((q, N_FF)) * 20
    gate[3 * q:] = rng.uniform(-12, 12, (rows - 3 * q, N_FF))
    up[3 * q:] = rng.uniform(-3, 3, (rows - 3 * q, N_FF))
    gate[0, :32], up[0, :32] = 1.25, -0.75                    # every value equal
    gate[1, :32], up[1, :32] = rng.standard_normal(32), 0.5
    gate[1, 5] = gate[1, 17] = 3.0                            # two tied maxima
    gate[2, :64], up[2, :64] = 0.0, 1.0                       # all-zero blocks
    gate[3, :32] = np.float32(1e-40)                          # subnormal gates
    gate[3, 32:64] = np.float32([1e30, -1e30] * 16)           # tanh = +-1, inner overflows
    up[4, :32] = np.float32(1e-39)                            # subnormal results
    gu = np.concatenate([gate, up], 1)
    gq, gd = qbuf(eg2, rows, N_FF, gpu), empty((36, rows), torch.float32, gpu)
    eg2.ops.gelu_quant(dev(gu, gpu), gq, gd)
    with np.errstate(all="ignore"):
        wq, wd = oracle_gelu_q8(gate, up)
    assert np.array_equal(bits(host(gd).T), bits(wd))
    got = qvals(eg2, gq, rows, N_FF)
    bad = np.argwhere(got != wq)
    assert bad.size == 0, (bad[:5], got[tuple(bad[0])], wq[tuple(bad[0])])


def test_device_libm_equals_host_libm(eg2, gpu):
    """The device's expf and tanhf (eg2_libm.hpp) against the host's libm
    on every 97th float bit pattern (44 million values: normal, subnormal,
    zero, infinite) plus every float in [-2, 2]'s coarse grid."""
    import torch

    u = np.arange(0, 1 << 32, 97, dtype=np.uint64).astype(np.uint32)
    x = u.view(np.float32)
    x = x[~np.isnan(x)]
    x = np.concatenate([x, np.linspace(-2, 2, 1 << 20, dtype=np.float32)])
    xd = dev(x, gpu)
    ed, td = torch.empty_like(xd), torch.empty_like(xd)
    eg2.check(eg2.lib().eg2_hip_libm_eval(eg2.ops._p(xd), x.size, eg2.ops._p(ed), eg2.ops._p(td), eg2.ops._stream()),
              "libm_eval")
    with np.errstate(all="ignore"):
        host_exp = OL.host_libm("expf", x)
        host_tanh = OL.host_libm("tanhf", x)
    assert np.array_equal(bits(host(ed)), bits(host_exp))
    assert np.array_equal(bits(host(td)), bits(host_tanh))


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
                                   (16, 3072, 768), (16, 768, 3072), (300, 768, 1152), (1, 32, 32),
                                   (70, 96, 320), (40, 64, 224)])
def test_gemm_q8_bit_exact(eg2, gpu, n, m, k):
    """Config 1 (512 x 2304 x 768) and every projection shape of the forward,
    and block counts that take the block loop's tail (10 and 7 blocks: one
    round of 6 and a remainder): identical to the reference's Q8_0 x Q8_0
    dot (gemma2.c:120-141)."""
    import torch

    w = quantize_q8_0((RNG.standard_normal((m, k)) * 0.02).astype(np.float32))
    xb = quantize_q8_0(RNG.standard_normal((n, k)).astype(np.float32))
    xb[0, 0]["qs"][:] = -128  # the most negative Q8_0 value round-trips too
    y = empty((n, m), torch.float32, gpu)
    eg2.ops.gemm_q8(*device_q8(eg2, xb, k, gpu), *device_weights(eg2, w, k, gpu), y)
    assert np.array_equal(host(y), OL.gemm_q8_0(w, xb))


def test_gemm_q8_extreme_block_dots(eg2, gpu):
    """Block dots at both ends of their range (all -128 x -128 = +2^19, and
    -128 x 127 = -16256 x 32) and scales across the fp16 range, subnormal
    to the largest (outputs from 1e-9 to 1e16): the biased accumulator
    keeps every dot exact (1.5 2^23 + dot stays in [2^23, 2^24)), and the
    outputs are the oracle's bit for bit."""
    import torch

    n, m, k = 64, 96, 768
    w = quantize_q8_0((RNG.standard_normal((m, k)) * 0.02).astype(np.float32))
    xb = quantize_q8_0(RNG.standard_normal((n, k)).astype(np.float32))
    w["qs"][: m // 2] = -128
    w["qs"][m // 2:m // 2 + 8] = 127
    xb["qs"][: n // 2] = -128
    scales = np.array([6.0e-8, 6.1e-5, 1.0, 0.0039, 1024.0, 65504.0], np.float16)
    w["d"] = scales[RNG.integers(0, len(scales), w["d"].shape)].view(np.uint16)
    xb["d"] = scales[RNG.integers(0, len(scales), xb["d"].shape)].view(np.uint16)
    w["d"][-8:] = scales[0].view(np.uint16)  # rows and columns of the smallest scale only
    xb["d"][-8:] = scales[0].view(np.uint16)
    y = empty((n, m), torch.float32, gpu)
    eg2.ops.gemm_q8(*device_q8(eg2, xb, k, gpu), *device_weights(eg2, w, k, gpu), y)
    want = OL.gemm_q8_0(w, xb)
    assert np.array_equal(bits(host(y)), bits(want))
    mag = np.abs(want[want != 0])
    assert mag.max() > 1e15 and mag.min() < 1e-6


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


def test_gemm_q8_geglu_tied_block_maxima(eg2, gpu):
    """Blocks whose largest GeGLU value occurs more than once (repeated
    weight rows): the first candidate of each block is evaluated in the
    workgroup's shared pass, the others in the per-wave passes. Block 0 has
    32 equal rows (every value a candidate, in all four lanes), block 1
    equal pairs (extra candidates in the owner lane), block 2 rows repeated
    16 apart (an extra candidate in another lane); the rest are random. Bit
    for bit the oracle's and the two-kernel path's."""
    import torch

    k, ff, n = N_EMBD, N_FF, 96
    wg = (RNG.standard_normal((ff, k)) * 0.02).astype(np.float32)
    wu = (RNG.standard_normal((ff, k)) * 0.02).astype(np.float32)
    for w in (wg, wu):
        w[1:32] = w[0]
        w[33:64:2] = w[32:64:2]
        w[80:96] = w[64:80]
    wg, wu = quantize_q8_0(wg), quantize_q8_0(wu)
    xb = quantize_q8_0(RNG.standard_normal((n, k)).astype(np.float32))
    q, d = run_geglu(eg2, gpu, xb, wg, wu, k, ff, n)
    wq, wd = oracle_gelu_q8(OL.gemm_q8_0(wg, xb), OL.gemm_q8_0(wu, xb))
    assert np.array_equal(q, wq)
    assert np.array_equal(bits(d.T), bits(wd))
    y = empty((n, 2 * ff), torch.float32, gpu)
    eg2.ops.gemm_q8(*device_q8(eg2, xb, k, gpu), *device_weights(eg2, np.concatenate([wg, wu]), k, gpu), y)
    rq, rd = qbuf(eg2, n, ff, gpu), empty((ff // 32, n), torch.float32, gpu)
    eg2.ops.gelu_quant(y, rq, rd)
    assert np.array_equal(q, qvals(eg2, rq, n, ff))
    assert np.array_equal(bits(d), bits(host(rd)))


@pytest.mark.parametrize("n,ff,k", [(64, 32, 32), (100, 96, 160), (65, 1152, 768), (40, 64, 448)])
def test_gemm_q8_geglu_against_oracle(eg2, gpu, n, ff, k):
    """Other widths (k = 160 and 448: 5 and 14 blocks, not multiples of the
    block loop's unrolling by 6, so the loop's tail runs, after no full
    round and after two): the projections, the GeGLU and its Q8_0 bit for
    bit the oracle's."""
    wg = quantize_q8_0((RNG.standard_normal((ff, k)) * 0.05).astype(np.float32))
    wu = quantize_q8_0((RNG.standard_normal((ff, k)) * 0.05).astype(np.float32))
    xb = quantize_q8_0(RNG.standard_normal((n, k)).astype(np.float32))
    q, d = run_geglu(eg2, gpu, xb, wg, wu, k, ff, n)
    wq, wd = oracle_gelu_q8(OL.gemm_q8_0(wg, xb), OL.gemm_q8_0(wu, xb))
    assert np.array_equal(q, wq)
    assert np.array_equal(bits(d.T), bits(wd))


@pytest.mark.parametrize("lens", [[128] * 16, [40, 260], [33], [1, 1, 5], [2048]])
def test_gemm_q8_qkv_rope_bit_exact(eg2, gpu, lens):
    """The fused QKV projection + QK-norm/RoPE of the forward equals the
    oracle's projection then ei_qk_norm_rope_qk_inplace bit for bit, and
    equals eg2_hip_gemm_q8 on [q|k|v] followed by eg2_hip_qk_norm_rope."""
    import torch

    k = N_EMBD
    n = int(sum(lens))
    w = quantize_q8_0((RNG.standard_normal((eg2.QKV_COLS, k)) * 0.05).astype(np.float32))
    xb = quantize_q8_0(RNG.standard_normal((n, k)).astype(np.float32))
    xq, xd = device_q8(eg2, xb, k, gpu)
    wq, wd = device_weights(eg2, w, k, gpu)
    qw, kw = ((1 + 0.1 * RNG.standard_normal(HEAD_DIM)).astype(np.float32) for _ in range(2))
    pos = np.concatenate([np.arange(l) for l in lens]).astype(np.int32)
    table = dev(eg2.rope_table(1e4), gpu)
    args = (dev(qw, gpu), dev(kw, gpu), table, dev(pos, gpu), 1e-6)
    fused = torch.full((n, eg2.QKV_COLS), 7.0, device=gpu)
    eg2.ops.gemm_q8_qkv_rope(xq, xd, wq, wd, n, *args, fused)
    y = empty((n, eg2.QKV_COLS), torch.float32, gpu)
    eg2.ops.gemm_q8(xq, xd, wq, wd, y)
    eg2.ops.qk_norm_rope(y, *args, y)
    want = oracle_qk_norm_rope(OL.gemm_q8_0(w, xb), qw, kw, pos, 1e4)
    assert np.array_equal(bits(host(fused)), bits(want))
    assert np.array_equal(bits(host(y)), bits(want))


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


def run_attention(eg2, gpu, q, k, v, offsets, window, scratch_fill=0.0, longest=None):
    """The device attention of rows [q | k | v] packed as `offsets` (rows
    padded to a multiple of 4 by one more sequence): (int8 [T, 768], scales
    [T, 24]) of the quantized context. longest: the softmax form override
    (None: the plan's longest sequence; 0: the form for any length)."""
    import torch

    T = q.shape[0]
    rows = (T + 3) // 4 * 4
    offs = list(np.asarray(offsets, np.int64)) + ([rows] if rows > T else [])
    qkv = np.zeros((rows, eg2.QKV_COLS), np.float32)
    qkv[:T] = np.concatenate([q, k, v], axis=1)
    cq, cd = qbuf(eg2, rows, N_EMBD, gpu), empty((24, rows), torch.float32, gpu)
    plan = eg2.AttentionPlan(offs, gpu, rows)
    plan.scores.fill_(scratch_fill)
    eg2.ops.attention_planned(dev(qkv, gpu), plan, window, cq, cd, longest)
    return qvals(eg2, cq, rows, N_EMBD)[:T], np.ascontiguousarray(host(cd).T)[:T]


def oracle_attention(q, k, v, offsets, window):
    """The oracle's attention per sequence (fp32 context)."""
    T = q.shape[0]
    ctx = np.zeros((T, N_EMBD), np.float32)
    sc = np.zeros(4096, np.float32)
    for s in range(len(offsets) - 1):
        a, b = int(offsets[s]), int(offsets[s + 1])
        oracle().or_attention_range(fptr(np.ascontiguousarray(q[a:b])), fptr(np.ascontiguousarray(k[a:b])),
                                    fptr(np.ascontiguousarray(v[a:b])), b - a, window, 0, b - a, fptr(ctx[a:b]),
                                    fptr(sc))
    return ctx


def assert_attention_bit_exact(cq, cd, ctx):
    wq, wd = split(quantize_q8_0(ctx), N_EMBD)
    assert np.array_equal(cq, wq)
    assert np.array_equal(bits(cd), bits(wd))


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


def qkv_inputs(rng, T):
    q = (rng.standard_normal((T, N_EMBD)) * 0.0625).astype(np.float32)
    k = rng.standard_normal((T, HEAD_DIM)).astype(np.float32)
    v = rng.standard_normal((T, HEAD_DIM)).astype(np.float32)
    return q, k, v


@pytest.mark.parametrize("window", [0, 512])
def test_attention_packed_bit_exact(eg2, gpu, window):
    """Config-2 shape: T=2048 packed from 16 log-uniform segments (8..512):
    the quantized context is the oracle's bit for bit (full attention and a
    512 window). The oracle's fp32 context itself is within 2^-16 max|v|
    of float64 attention."""
    rng = np.random.default_rng(2)
    lens = segments_log_uniform(rng)
    T = int(lens.sum())
    offsets = np.concatenate([[0], np.cumsum(lens)])
    q, k, v = qkv_inputs(rng, T)
    cq, cd = run_attention(eg2, gpu, q, k, v, offsets, window)
    ctx = oracle_attention(q, k, v, offsets, window)
    assert np.abs(ctx - attention_double(q, k, v, offsets, window)).max() <= 2.0 ** -16 * np.abs(v).max()
    assert_attention_bit_exact(cq, cd, ctx)


@pytest.mark.parametrize("lens,window", [([1100, 600, 300, 48], 0), ([2048], 0), ([700, 5, 900], 64),
                                         ([30, 31, 3], 1), ([17, 40], 2), ([2500, 52], 0), ([2600], 512)])
def test_attention_long_and_windowed_bit_exact(eg2, gpu, lens, window):
    """Long sequences (many 64-key blocks and query chunks, and rows past
    the 2048 keys of an executor wave: ten chunks of the softmax's LDS ring)
    and narrow windows (down to the token and its neighbours): the oracle's
    bits."""
    rng = np.random.default_rng(sum(lens) + window)
    T = sum(lens)
    offsets = np.concatenate([[0], np.cumsum(lens)])
    q, k, v = qkv_inputs(rng, T)
    cq, cd = run_attention(eg2, gpu, q, k, v, offsets, window)
    assert_attention_bit_exact(cq, cd, oracle_attention(q, k, v, offsets, window))


def test_attention_single_token_segments(eg2, gpu):
    """Length-1 sequences attend only to themselves: p = expf(0) = 1, so the
    context is v exactly, quantized like the reference."""
    T = 64
    q = RNG.standard_normal((T, N_EMBD)).astype(np.float32)
    k = RNG.standard_normal((T, HEAD_DIM)).astype(np.float32)
    v = RNG.standard_normal((T, HEAD_DIM)).astype(np.float32)
    cq, cd = run_attention(eg2, gpu, q, k, v, np.arange(T + 1), 0)
    wq, wd = split(quantize_q8_0(np.tile(v, (1, 3))), N_EMBD)
    assert np.array_equal(cq, wq) and np.array_equal(bits(cd), bits(wd))


@pytest.mark.parametrize("window", [0, 16])
def test_attention_independent_of_packing(eg2, gpu, window):
    """A sequence gives bit-identical context alone or anywhere in a wave."""
    rng = np.random.default_rng(8)
    lens = [37, 5, 64, 1, 100, 33]
    T = sum(lens)
    offsets = np.concatenate([[0], np.cumsum(lens)])
    q, k, v = qkv_inputs(rng, T)
    cq, cd = run_attention(eg2, gpu, q, k, v, offsets, window)
    for s in range(len(lens)):
        a, b = offsets[s], offsets[s + 1]
        sq, sd = run_attention(eg2, gpu, q[a:b], k[a:b], v[a:b], [0, b - a], window)
        assert np.array_equal(sq, cq[a:b]) and np.array_equal(sd, cd[a:b])


@pytest.mark.parametrize("window", [0, 64])
@pytest.mark.parametrize("lens", [[1, 130, 512, 7, 300], [1, 513, 2, 1200, 37]])
def test_attention_softmax_forms_agree(eg2, gpu, window, lens):
    """The softmax forms (16 or 32 lanes per pair for waves of sequences up
    to 128 or 256 tokens, a wave per pair up to 512, rows streamed through
    an LDS ring for any length) give the same bits, and so does a `longest`
    below the wave's real longest sequence (rows too long for the chosen
    form's LDS are summed from global memory): the hint picks a kernel form,
    never the results."""
    rng = np.random.default_rng(10 + len(lens))
    T = sum(lens)
    offsets = np.concatenate([[0], np.cumsum(lens)])
    q, k, v = qkv_inputs(rng, T)
    ref = run_attention(eg2, gpu, q, k, v, offsets, window)
    for longest in (h for h in (0, 1, 128, 129, 256, 257, 512, 513, 2048) if h <= T):
        got = run_attention(eg2, gpu, q, k, v, offsets, window, longest=longest)
        assert np.array_equal(ref[0], got[0]) and np.array_equal(bits(ref[1]), bits(got[1])), longest
    assert_attention_bit_exact(*ref, oracle_attention(q, k, v, offsets, window))


@pytest.mark.parametrize("lens", [[128] * 8 + [60, 4], [700, 5, 300, 39]])
def test_attention_any_grid_same_bits(eg2, gpu, lens):
    """The workgroups take the items XCD by XCD (a contiguous eighth each)
    when the grid is a multiple of 8 and stride over the whole list
    otherwise; a small grid walks many items per workgroup. Grids 8, 61, 1
    and 1024 give the same bits, for short waves (the context kernel in XCD
    order too) and long ones."""
    import torch

    rng = np.random.default_rng(14 + len(lens))
    T = sum(lens)
    offsets = np.concatenate([[0], np.cumsum(lens)])
    q, k, v = qkv_inputs(rng, T)
    ref = run_attention(eg2, gpu, q, k, v, offsets, 0)
    rows = (T + 3) // 4 * 4
    offs = list(offsets) + ([rows] if rows > T else [])
    qkv = np.zeros((rows, eg2.QKV_COLS), np.float32)
    qkv[:T] = np.concatenate([q, k, v], axis=1)
    for grid in (8, 61, 1):
        plan = eg2.AttentionPlan(offs, gpu, rows)
        plan.GRID = grid
        cq, cd = qbuf(eg2, rows, N_EMBD, gpu), empty((24, rows), torch.float32, gpu)
        eg2.ops.attention_planned(dev(qkv, gpu), plan, 0, cq, cd)
        got = qvals(eg2, cq, rows, N_EMBD)[:T], np.ascontiguousarray(host(cd).T)[:T]
        assert np.array_equal(got[0], ref[0]) and np.array_equal(bits(got[1]), bits(ref[1])), grid


@pytest.mark.parametrize("lens", [[128] * 16, [2048], [1, 513, 2, 1200, 37]])
def test_attention_stages_equal_the_whole(eg2, gpu, lens):
    """eg2_hip_attention_scores, _softmax and _context launched one by one
    (how the profile and the benchmark time them) give eg2_hip_attention's
    bits."""
    import torch

    rng = np.random.default_rng(20 + len(lens))
    T = sum(lens)
    offsets = np.concatenate([[0], np.cumsum(lens)])
    q, k, v = qkv_inputs(rng, T)
    ref = run_attention(eg2, gpu, q, k, v, offsets, 0)
    rows = (T + 3) // 4 * 4
    offs = list(offsets) + ([rows] if rows > T else [])
    qkv = np.zeros((rows, eg2.QKV_COLS), np.float32)
    qkv[:T] = np.concatenate([q, k, v], axis=1)
    qkv_d = dev(qkv, gpu)
    plan = eg2.AttentionPlan(offs, gpu, rows)
    cq, cd = qbuf(eg2, rows, N_EMBD, gpu), empty((24, rows), torch.float32, gpu)
    for stage in ("scores", "softmax", "context"):
        eg2.ops.attention_stage(stage, qkv_d, plan, 0, cq, cd)
    got = qvals(eg2, cq, rows, N_EMBD)[:T], np.ascontiguousarray(host(cd).T)[:T]
    assert np.array_equal(got[0], ref[0]) and np.array_equal(bits(got[1]), bits(ref[1]))


def test_attention_reads_only_scores_it_wrote(eg2, gpu):
    """The scores scratch is written before it is read: any prior content
    (zeros, huge values, NaN) gives the same bits."""
    rng = np.random.default_rng(9)
    lens = [3, 40, 1, 70, 129]
    T = sum(lens)
    offsets = np.concatenate([[0], np.cumsum(lens)])
    q, k, v = qkv_inputs(rng, T)
    a = run_attention(eg2, gpu, q, k, v, offsets, 0, scratch_fill=0.0)
    for fill in (1e30, float("nan")):
        b = run_attention(eg2, gpu, q, k, v, offsets, 0, scratch_fill=fill)
        assert np.array_equal(a[0], b[0]) and np.array_equal(bits(a[1]), bits(b[1]))


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


def test_config3_layer_through_the_operators_bit_exact(eg2, gpu):
    """Configuration 3 as specified: one encoder layer over configuration
    2's 16 log-uniform segments, hidden state ~ N(0,1), weights N(0, 0.02)
    -> Q8_0, through the operator entry points in the executor's kernel
    order (bench.DeviceLayer). The residual stream after the layer is the
    oracle's layer_forward bit for bit, run twice in a row (the second from
    the same input), and the Q8_0 activations it leaves for the next layer
    are the oracle quantizer's of attn_norm(x)."""
    import bench

    rng = np.random.default_rng(0)
    lens = bench.segments_log_uniform(rng)
    offsets = np.concatenate([[0], np.cumsum(lens)])
    T = int(offsets[-1])
    x0 = rng.standard_normal((T, N_EMBD)).astype(np.float32)
    L = bench.layer_weights(rng)
    lay = bench.DeviceLayer(eg2, __import__("torch"), L, offsets)
    want = OL.layer_forward(L, x0, offsets, 1e4, 0, 1e-6, 16)
    for _ in range(2):
        lay.prepare(x0)
        lay.run()
        got = lay.x.cpu().numpy()
        assert np.array_equal(got, want)
    nxt = np.zeros((T, N_EMBD // 32), Q8)
    want = np.ascontiguousarray(want)
    for t in range(T):
        oracle().or_rms_norm_quantize_q8_0(fptr(want[t]), fptr(L["attn_norm"]), N_EMBD, 1e-6, vptr(nxt[t]))
    q = qvals(eg2, lay.xq[:eg2.q8_tile_bytes(T, N_EMBD)], T, N_EMBD)
    d = np.ascontiguousarray(host(lay.xd[:24]).T)
    wq, wd = split(nxt, N_EMBD)
    assert np.array_equal(q, wq) and np.array_equal(bits(d), bits(wd))
