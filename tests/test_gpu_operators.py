"""The operator kernels that take the include/abi.h records
(kernels_abi.hip: MFMA projections, chunked attention, register-row norms),
launched by name through eg2_op_launch with the grids and workgroup sizes
of the reference's operator test, tests/kernels.cpp, and once from the
stand-alone code object through hipModuleLoad.

Cases and tolerances follow tests/kernels.cpp:
  * projections (:57-80): four tilings x four weight types x n in
    {1, 17, 33, 65}, k 64, m 35, inputs whose every partial sum is exact, so
    the check is bit-exact; plus random inputs over several K slices against
    a float64 product, within 4e-6 of the sum of |x w|;
  * norm (:81-91) against a float64 sum of squares, 2e-5;
  * fused vs unfused (:92-113): norm_residual = norm + element(mode 0), and
    norm_rope = norm + rope, 2e-6;
  * attention (:114-137): GQA, two sequences, SWA window 1, against a
    float64 softmax, 2e-5; plus the 3-query-head variant the same way, with
    sequences longer than one 64-key chunk.
Also: the gathers and pooling bit-exact against float32 restatements,
element modes 1/2 against float64 gelu_tanh, saxpy on exact inputs."""
import math

import numpy as np
import pytest

import oracle_lib as OL

pytestmark = pytest.mark.gpu


def dev(a, gpu):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def ptr(t):
    return t.data_ptr()


# --------------------------------------------------------------- projections

MM_VARIANTS = [("eg2_mm", 16, 16, 16), ("eg2_mm64", 64, 16, 32), ("eg2_mm64x64", 64, 64, 32),
               ("eg2_mmstep8", 64, 64, 8)]  # name, tile width (m), tile height (n), k step


def encode_weights(w, wtype):
    """fp32 [m, k] -> the GGML layout of type 0/1/8/30 (Q8_0 blocks run over
    the flattened matrix) and the decoded fp32 values the kernel sees."""
    flat = w.reshape(-1)
    if wtype == 0:
        return flat.astype(np.float32).view(np.uint8), w.astype(np.float32)
    if wtype == 1:
        h = flat.astype(np.float16)
        return h.view(np.uint8), h.astype(np.float32).reshape(w.shape)
    if wtype == 30:
        bits = (flat.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        return bits.view(np.uint8), (bits.astype(np.uint32) << 16).view(np.float32).reshape(w.shape)
    assert wtype == 8
    nblk = (flat.size + 31) // 32
    padded = np.zeros(nblk * 32, np.float32)
    padded[: flat.size] = flat
    blocks = OL.quantize_q8_0(padded.reshape(1, -1))[0]
    dec = OL.dequantize_q8_0(blocks.reshape(1, -1)).reshape(-1)[: flat.size]
    return blocks.view(np.uint8), dec.reshape(w.shape)


def run_mm(eg2, gpu, name, width, height, x, raw_w, wtype, m):
    import torch

    n, k = x.shape
    xd = dev(x, gpu)
    wd = dev(raw_w, gpu)
    yd = torch.full((n, m), float("nan"), dtype=torch.float32, device=gpu)
    rec = eg2.EgMM(ptr(yd), ptr(xd), ptr(wd), n, k, m, wtype)
    eg2.ops.op(name, rec, ((m + width - 1) // width, (n + height - 1) // height), 256)
    return host(yd)


@pytest.mark.parametrize("variant", MM_VARIANTS, ids=[v[0] for v in MM_VARIANTS])
@pytest.mark.parametrize("wtype", [0, 1, 8, 30])
def test_mm_exact_cases(eg2, gpu, variant, wtype):
    """tests/kernels.cpp:57-80: x = (i%19 - 9)/32, w = (i%23 - 11)/8 (as Q8_0:
    d = 0.125, q = i%23 - 11). Every product and partial sum is exact."""
    name, width, height, _ = variant
    k, m = 64, 35
    w = ((np.arange(k * m) % 23) - 11).astype(np.float32).reshape(m, k) * 0.125
    if wtype == 8:
        raw = np.zeros(k * m // 32, OL.Q8)
        raw["d"] = 0x3000  # fp16 0.125
        raw["qs"] = (((np.arange(k * m) % 23) - 11).reshape(-1, 32)).astype(np.int8)
        raw = raw.view(np.uint8)
    else:
        raw, dec = encode_weights(w, wtype)
        assert np.array_equal(dec, w)
    for n in (1, 17, 33, 65):
        x = ((np.arange(n * k) % 19) - 9).astype(np.float32).reshape(n, k) * 0.03125
        want = (x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32)
        got = run_mm(eg2, gpu, name, width, height, x, raw, wtype, m)
        assert np.array_equal(got, want), (name, wtype, n)


@pytest.mark.parametrize("variant", MM_VARIANTS, ids=[v[0] for v in MM_VARIANTS])
@pytest.mark.parametrize("wtype", [0, 1, 8, 30])
@pytest.mark.parametrize("shape", [(37, 70, 67), (130, 770, 200)])
def test_mm_random_against_float64(eg2, gpu, variant, wtype, shape):
    """Random inputs, k not a multiple of the 32-value slice, partial tiles
    in both directions: within 4e-6 of sum |x w| of the float64 product of
    the decoded weights (a wrong operand or output placement is off by O(1))."""
    name, width, height, _ = variant
    rng = np.random.default_rng(7 + wtype + shape[1])
    n, k, m = shape
    x = rng.standard_normal((n, k)).astype(np.float32)
    raw, dec = encode_weights((rng.standard_normal((m, k)) * 0.05).astype(np.float32), wtype)
    got = run_mm(eg2, gpu, name, width, height, x, raw, wtype, m)
    x64, w64 = x.astype(np.float64), dec.astype(np.float64)
    want, mag = x64 @ w64.T, np.abs(x64) @ np.abs(w64).T
    assert np.all(np.abs(got - want) <= 4e-6 * mag + 1e-30), np.abs(got - want).max()


def test_code_object_dispatch_by_name(eg2, gpu):
    """The stand-alone code object eg2_ops_gfx950.co, loaded with
    hipModuleLoad and eg2_mm64x64 launched by symbol name with the EgMM
    record as its kernarg buffer (src/gemma2_kfd.cpp:106-110, 156-170):
    the same output as the library's own launch of the operator."""
    import ctypes as C
    import os

    import torch

    hip = C.CDLL("libamdhip64.so.7")  # the runtime already in the process
    co = os.path.join(os.path.dirname(eg2.LIB_PATH), "eg2_ops_gfx950.co")
    assert os.path.exists(co)
    mod, fn = C.c_void_p(), C.c_void_p()
    assert hip.hipModuleLoad(C.byref(mod), co.encode()) == 0
    try:
        assert hip.hipModuleGetFunction(C.byref(fn), mod, b"eg2_mm64x64") == 0
        rng = np.random.default_rng(3)
        n, k, m = 70, 96, 130
        x = rng.standard_normal((n, k)).astype(np.float32)
        raw, dec = encode_weights((rng.standard_normal((m, k)) * 0.05).astype(np.float32), 8)
        xd, wd = dev(x, gpu), dev(raw, gpu)
        y = torch.full((n, m), float("nan"), dtype=torch.float32, device=gpu)
        rec = eg2.EgMM(ptr(y), ptr(xd), ptr(wd), n, k, m, 8)
        size = C.c_size_t(C.sizeof(rec))
        extra = (C.c_void_p * 5)(1, C.addressof(rec), 2, C.addressof(size), 3)  # BUFFER_POINTER, SIZE, END
        stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        hip.hipModuleLaunchKernel.argtypes = [C.c_void_p] + [C.c_uint] * 7 + [C.c_void_p, C.c_void_p, C.c_void_p]
        assert hip.hipModuleLaunchKernel(fn, (m + 63) // 64, (n + 63) // 64, 1, 256, 1, 1, 0, stream, None,
                                         extra) == 0
        got = host(y)
    finally:
        torch.cuda.synchronize()
        assert hip.hipModuleUnload(mod) == 0
    same = run_mm(eg2, gpu, "eg2_mm64x64", 64, 64, x, raw, 8, m)
    assert np.array_equal(got, same)
    want = x.astype(np.float64) @ dec.astype(np.float64).T
    assert np.abs(got - want).max() <= 4e-6 * (np.abs(x) @ np.abs(dec).T).max()


# ------------------------------------------------------------------- norms

def test_norm_against_float64(eg2, gpu):
    """tests/kernels.cpp:81-91."""
    import torch

    for d in (256, 512):
        w = (0.5 + (np.arange(d) % 7) * 0.1).astype(np.float32)
        x = np.sin(np.arange(3 * d, dtype=np.float32) * np.float32(0.13)).astype(np.float32).reshape(3, d)
        xd, wd = dev(x, gpu), dev(w, gpu)
        yd = torch.zeros((3, d), dtype=torch.float32, device=gpu)
        eg2.ops.op("eg2_norm", eg2.EgNorm(ptr(yd), ptr(xd), ptr(wd), 3, d, 1.0), 3, 64)
        got = host(yd)
        ss = (x.astype(np.float64) ** 2).sum(1, keepdims=True)
        want = x * w / np.sqrt((ss / d).astype(np.float32) + np.float32(1e-6))
        assert np.abs(got - want).max() <= 2e-5


def test_norm_scale_and_null_weight(eg2, gpu):
    """EgNorm.scale pre-scales x (kernels/eg2.c:127); weight NULL means 1."""
    import torch

    d = 768
    x = np.random.default_rng(2).standard_normal((5, d)).astype(np.float32)
    xd = dev(x, gpu)
    yd = torch.zeros((5, d), dtype=torch.float32, device=gpu)
    eg2.ops.op("eg2_norm", eg2.EgNorm(ptr(yd), ptr(xd), None, 5, d, 0.25), 5, 64)
    xs = x.astype(np.float64) * 0.25
    want = xs / np.sqrt((xs ** 2).mean(1, keepdims=True) + 1e-6)
    assert np.abs(host(yd) - want).max() <= 2e-5
    # in place
    eg2.ops.op("eg2_norm", eg2.EgNorm(ptr(xd), ptr(xd), None, 5, d, 0.25), 5, 64)
    assert np.array_equal(host(xd), host(yd))


def test_fused_matches_unfused(eg2, gpu):
    """tests/kernels.cpp:92-113: norm_residual == norm + element(mode 0), and
    norm_rope == norm + rope, including in-place aliases and per-token
    tables."""
    import torch

    for d in (256, 512):
        w = (0.5 + (np.arange(d) % 7) * 0.1).astype(np.float32)
        i = np.arange(6 * d, dtype=np.float32)
        x = np.sin(i * np.float32(0.13)).astype(np.float32)
        res = np.cos(i * np.float32(0.17)).astype(np.float32)
        xd, wd, resd, saved = dev(x, gpu), dev(w, gpu), dev(res, gpu), dev(res.copy(), gpu)
        y = torch.zeros(6 * d, dtype=torch.float32, device=gpu)
        eg2.ops.op("eg2_norm", eg2.EgNorm(ptr(y), ptr(xd), ptr(wd), 6, d, 1.0), 6, 64)
        eg2.ops.op("eg2_element", eg2.EgElement(ptr(resd), ptr(resd), ptr(y), 6 * d, 0, 0, 0.7),
                   (6 * d + 255) // 256, 256)
        eg2.ops.op("eg2_norm_residual", eg2.EgNormResidual(ptr(saved), ptr(xd), ptr(wd), 6, d, 0.7), 6, 64)
        assert np.abs(host(saved) - host(resd)).max() <= 2e-6

        table = np.zeros(3 * d, np.float32)
        for t in range(3):
            z = np.arange(d // 2, dtype=np.float32)
            table[t * d: t * d + d // 2] = np.cos(np.float32(t) * z * np.float32(0.01))
            table[t * d + d // 2: (t + 1) * d] = np.sin(np.float32(t) * z * np.float32(0.01))
        td = dev(table, gpu)
        eg2.ops.op("eg2_norm", eg2.EgNorm(ptr(y), ptr(xd), ptr(wd), 6, d, 1.0), 6, 64)
        eg2.ops.op("eg2_rope", eg2.EgRope(ptr(y), ptr(td), 3, 2, d), (6 * d // 2 + 255) // 256, 256)
        eg2.ops.op("eg2_norm_rope", eg2.EgNormRope(ptr(xd), ptr(wd), ptr(td), 6, d, 2), 6, 64)
        assert np.abs(host(xd) - host(y)).max() <= 2e-6


# ---------------------------------------------------------------- attention

def attention_reference(q, k, v, bounds, n, heads, d, kv_stride, kh_of, window):
    out = np.zeros((n * heads, d))
    for t in range(n):
        for h in range(heads):
            lo, hi = int(bounds[2 * t]), int(bounds[2 * t + 1])
            if window:
                if t > window:
                    lo = max(lo, t - window)
                hi = min(hi, t + window + 1)
            kh = kh_of(h)
            qv = q[(t * heads + h) * d:(t * heads + h + 1) * d].astype(np.float64)
            keys = np.stack([k[s * kv_stride + kh * d: s * kv_stride + (kh + 1) * d] for s in range(lo, hi)])
            vals = np.stack([v[s * kv_stride + kh * d: s * kv_stride + (kh + 1) * d] for s in range(lo, hi)])
            sc = np.exp(keys.astype(np.float64) @ qv)
            out[t * heads + h] = (sc / sc.sum()) @ vals.astype(np.float64)
    return out


@pytest.mark.parametrize("d", [256, 512])
@pytest.mark.parametrize("window", [0, 1])
def test_attention_against_float64(eg2, gpu, d, window):
    """tests/kernels.cpp:114-137: 8 tokens in sequences [0,3) and [3,8)."""
    import torch

    bounds = np.array([v for t in range(8) for v in ((0, 3) if t < 3 else (3, 8))], np.uint32)
    q = (np.sin(np.arange(8 * 2048, dtype=np.float32) * np.float32(0.07)) * np.float32(0.1)).astype(np.float32)
    i = np.arange(8 * 512, dtype=np.float32)
    k = (np.cos(i * np.float32(0.11)) * np.float32(0.1)).astype(np.float32)
    v = np.sin(i * np.float32(0.03)).astype(np.float32)
    qd, kd, vd, bd = dev(q, gpu), dev(k, gpu), dev(v, gpu), dev(bounds.view(np.int32), gpu)
    y = torch.zeros(8 * 4 * d, dtype=torch.float32, device=gpu)
    name = "eg2_attention256" if d == 256 else "eg2_attention512"
    eg2.ops.op(name, eg2.EgAttention(ptr(y), ptr(qd), ptr(kd), ptr(vd), ptr(bd), 8, window), 8 * 4, 64)
    per = 4 // (512 // d)
    want = attention_reference(q, k, v, bounds, 8, 4, d, 512, lambda h: h // per, window)
    assert np.abs(host(y).reshape(32, d) - want).max() <= 2e-5


@pytest.mark.parametrize("window", [0, 2, 50])
@pytest.mark.parametrize("lens", [[1, 6, 13], [70, 1, 150]])
def test_attention_3q1kv_against_float64(eg2, gpu, window, lens):
    """eg2_attention256x3: 3 query heads share the one KV head of 256;
    sequences longer than a 64-key chunk take the rescaling between chunks."""
    import torch

    rng = np.random.default_rng(5 + len(lens) + lens[0])
    n = sum(lens)
    starts = np.concatenate([[0], np.cumsum(lens)])
    bounds = np.array([v for s in range(len(lens)) for _ in range(lens[s]) for v in (starts[s], starts[s + 1])],
                      np.uint32)
    q = (rng.standard_normal(n * 3 * 256) * 0.1).astype(np.float32)
    k = (rng.standard_normal(n * 256) * 0.1).astype(np.float32)
    v = rng.standard_normal(n * 256).astype(np.float32)
    qd, kd, vd, bd = dev(q, gpu), dev(k, gpu), dev(v, gpu), dev(bounds.view(np.int32), gpu)
    y = torch.zeros(n * 3 * 256, dtype=torch.float32, device=gpu)
    eg2.ops.op("eg2_attention256x3", eg2.EgAttention(ptr(y), ptr(qd), ptr(kd), ptr(vd), ptr(bd), n, window),
               3 * n, 64)
    want = attention_reference(q, k, v, bounds, n, 3, 256, 256, lambda h: 0, window)
    assert np.abs(host(y).reshape(n * 3, 256) - want).max() <= 2e-5


# -------------------------------------------------------- elementwise, pool

def test_gathers_bit_exact(eg2, gpu):
    import torch

    rng = np.random.default_rng(11)
    for name, width, scale_first in (("eg2_gather", 512, False), ("eg2_gather768", 768, True)):
        rows = 40
        table = OL.quantize_q8_0((rng.standard_normal((rows, width)) * 0.05).astype(np.float32))
        ids = rng.integers(0, rows, 9).astype(np.int32)
        td, idd = dev(table.view(np.uint8), gpu), dev(ids, gpu)
        y = torch.zeros(9 * width, dtype=torch.float32, device=gpu)
        eg2.ops.op(name, eg2.EgGather(ptr(y), ptr(td), ptr(idd), 9), (9 * width + 255) // 256, 256)
        d = table["d"].view(np.float16).astype(np.float32)[ids]            # [9, width/32]
        q = table["qs"].astype(np.float32)[ids]                             # [9, width/32, 32]
        if scale_first:
            # the 768-wide CPU path: (d * sqrt(768)) * q, engine.c:288-295
            want = (d * np.float32(math.sqrt(768.0)))[:, :, None] * q
            got_oracle = np.zeros((9, width), np.float32)
            for r, i in enumerate(ids):
                OL.oracle().or_dequantize_row_q8_0_scaled(OL.vptr(table[i]), width, np.float32(math.sqrt(768.0)),
                                                          OL.fptr(got_oracle[r]))
            assert np.array_equal(got_oracle.reshape(9, -1, 32), want)
        else:
            want = (d[:, :, None] * q) * np.float32(22.62741699796952)
        assert np.array_equal(host(y).reshape(9, -1, 32), want.astype(np.float32)), name


def test_element_modes(eg2, gpu):
    import torch

    rng = np.random.default_rng(12)
    n = 3 * 512
    x = (rng.standard_normal(n) * 2).astype(np.float32)
    other = rng.standard_normal(n * 24).astype(np.float32)
    xd, od = dev(x, gpu), dev(other, gpu)
    y = torch.zeros(n, dtype=torch.float32, device=gpu)
    eg2.ops.op("eg2_element", eg2.EgElement(ptr(y), ptr(xd), ptr(od), n, 0, 0, 0.7), (n + 255) // 256, 256)
    assert np.array_equal(host(y), (x + other[:n]) * np.float32(0.7))
    xx = x.astype(np.float64)
    gelu = 0.5 * xx * (1 + np.tanh(math.sqrt(2 / math.pi) * (xx + 0.044715 * xx ** 3)))
    eg2.ops.op("eg2_element", eg2.EgElement(ptr(y), ptr(xd), ptr(od), n, 1, 0, 1.0), (n + 255) // 256, 256)
    assert np.abs(host(y) - gelu * other[:n]).max() <= 2e-6 * np.abs(other[:n]).max() * 4
    layer = 5
    gate = other[((np.arange(n) // 512) * 24 + layer) * 512 + np.arange(n) % 512]
    eg2.ops.op("eg2_element", eg2.EgElement(ptr(y), ptr(xd), ptr(od), n, 2, layer, 1.0), (n + 255) // 256, 256)
    assert np.abs(host(y) - gelu * gate).max() <= 2e-6 * np.abs(gate).max() * 4


def test_pool_bit_exact(eg2, gpu):
    import torch

    rng = np.random.default_rng(13)
    offsets = np.array([0, 1, 5, 60, 61], np.uint32)
    x = rng.standard_normal((61, 768)).astype(np.float32)
    xd, od = dev(x, gpu), dev(offsets.view(np.int32), gpu)
    y = torch.zeros((4, 768), dtype=torch.float32, device=gpu)
    eg2.ops.op("eg2_pool", eg2.EgPool(ptr(y), ptr(xd), ptr(od), 4), (4 * 768 + 255) // 256, 256)
    want = np.zeros((4, 768), np.float32)
    for s in range(4):
        acc = np.zeros(768, np.float32)
        for t in range(offsets[s], offsets[s + 1]):
            acc = acc + x[t]
        want[s] = acc / np.float32(offsets[s + 1] - offsets[s])
    assert np.array_equal(host(y), want)


def test_saxpy_exact(eg2, gpu):
    import torch

    n = 1000
    x = ((np.arange(n) % 37) - 18).astype(np.float32) / 64
    yv = ((np.arange(n) % 11) - 5).astype(np.float32) / 8
    xd, yd = dev(x, gpu), dev(yv.copy(), gpu)
    eg2.ops.op("eg2_saxpy", eg2.EgSaxpy(ptr(yd), ptr(xd), 1.5, n), (n + 255) // 256, 256)
    assert np.array_equal(host(yd), np.float32(1.5) * x + yv)


def test_rejects_bad_launch_shapes_on_device(eg2, gpu):
    import torch

    y = torch.zeros(16, dtype=torch.float32, device=gpu)
    rec = eg2.EgNorm(ptr(y), ptr(y), None, 1, 16, 1.0)
    with pytest.raises(eg2.HipError):
        eg2.ops.op("eg2_norm", rec, 1, 128)  # one wave per row
    with pytest.raises(eg2.HipError):
        eg2.ops.op("eg2_mm", eg2.EgMM(ptr(y), ptr(y), ptr(y), 1, 4, 4, 2), 1, 256)  # Q4_0 id
