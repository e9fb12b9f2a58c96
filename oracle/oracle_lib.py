"""ctypes bindings for the CPU oracle (oracle/liboracle.so) and, when it was
built from the reference tree, the compiled reference (oracle/_ref/libref.so).

Test infrastructure only (tests/, the smoke check and the CPU-baseline leg
of bench.py): the product path never imports this module.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libref.so")

N_EMBD, N_FF, N_HEAD, HEAD_DIM, N_CTX, VOCAB, QK = 768, 1152, 3, 256, 2048, 262144, 32
DENSE_FF = 3072

# GGUF Q8_0 block (quants.h:13-19): packed 34 bytes.
Q8 = np.dtype([("d", "<u2"), ("qs", "i1", (32,))])
assert Q8.itemsize == 34

_f = C.POINTER(C.c_float)
_i32 = C.POINTER(C.c_int32)
_vp = C.c_void_p


def fptr(a):
    return a.ctypes.data_as(_f)


def vptr(a):
    return C.c_void_p(a.ctypes.data)


def _load_oracle():
    if not os.path.exists(ORACLE_SO):
        raise RuntimeError("oracle/liboracle.so is not built (run `make -C oracle`)")
    lib = C.CDLL(ORACLE_SO)
    sig = {
        "or_fp32_to_fp16": (C.c_uint16, [C.c_float]),
        "or_fp16_to_fp32": (C.c_float, [C.c_uint16]),
        "or_quantize_row_q8_0": (None, [_f, _vp, C.c_int32]),
        "or_dequantize_row_q8_0_scaled": (None, [_vp, C.c_int32, C.c_float, _f]),
        "or_sum_squares": (C.c_float, [_f, C.c_int32]),
        "or_dot_f32": (C.c_float, [_f, _f, C.c_int32]),
        "or_rms_norm": (None, [_f, _f, C.c_int32, C.c_float, _f]),
        "or_rms_norm_quantize_q8_0": (None, [_f, _f, C.c_int32, C.c_float, _vp]),
        "or_rms_norm_residual_inplace": (None, [_f, _f, _f, C.c_int32, C.c_float]),
        "or_rope_cos_sin": (None, [C.c_int32, C.c_float, _f, _f]),
        "or_qk_norm_rope_qk_inplace": (None, [_f, _f, _f, _f, C.c_int32, C.c_float, C.c_float]),
        "or_attention_range": (None, [_f, _f, _f, C.c_int32, C.c_int32, C.c_int32, C.c_int32, _f, _f]),
        "or_gelu_tanh": (C.c_float, [C.c_float]),
        "or_gelu_mul_quantize_q8_0": (None, [_f, _f, C.c_int32, _vp]),
        "or_l2_normalize": (None, [_f, C.c_int32]),
        "or_normalize_prefix": (C.c_int, [_f, C.c_int32]),
        "or_mean_pool_rms": (None, [_f, C.c_int32, _f, C.c_float, _f]),
        "or_mean_pool_rms_l2": (None, [_f, C.c_int32, _f, C.c_float, _f]),
        "or_gemm_q8_0": (None, [_vp, _vp, C.c_int32, C.c_int32, C.c_int32, _f, C.c_int32]),
        "or_layer_forward": (None, [_vp, C.c_float, _f, _i32, _vp, C.c_size_t, C.c_int32]),
        "or_forward": (C.c_int, [_vp, _i32, _vp, C.c_size_t, _f, C.c_int32]),
        "or_libm_eval": (None, [_f, C.c_size_t, _f, _f]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def _load_ref():
    if not os.path.exists(REF_SO):
        return None
    lib = C.CDLL(REF_SO)
    sig = {
        "ei_fp32_to_fp16": (C.c_uint16, [C.c_float]),
        "ei_quantize_row_q8_0": (None, [_f, _vp, C.c_int32]),
        "ei_rms_norm": (None, [_f, _f, C.c_int32, C.c_float, _f]),
        "ei_rms_norm_quantize_q8_0": (None, [_f, _f, C.c_int32, C.c_float, _vp]),
        "ei_rms_norm_residual_inplace": (None, [_f, _f, _f, C.c_int32, C.c_float]),
        "ei_qk_norm_rope_qk_inplace": (None, [_f, _f, _f, _f, C.c_int32, C.c_float, C.c_float]),
        "ei_attention_mha_range": (None, [_f, _f, _f, C.c_int32, C.c_int32, C.c_int32, C.c_int32, _f, _f]),
        "ei_gelu_tanh": (C.c_float, [C.c_float]),
        "ei_gelu_mul_quantize_q8_0": (None, [_f, _f, C.c_int32, _vp]),
        "ei_l2_normalize": (None, [_f, C.c_int32]),
        "ei_embedding_normalize_prefix": (C.c_bool, [_f, C.c_int32]),
        "ei_mean_pool_rms_l2": (None, [_f, C.c_int32, _f, C.c_float, _f]),
        "ref_mm_q8_0": (None, [_vp, C.c_int, C.c_int, _f, C.c_int, _f]),
        "ref_embed_row": (None, [_vp, C.c_int, C.c_int, _f]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_oracle = None
_ref = None
_ref_loaded = False


def oracle():
    global _oracle
    if _oracle is None:
        _oracle = _load_oracle()
    return _oracle


def ref():
    """The compiled reference, or None where it was not built (GPU box)."""
    global _ref, _ref_loaded
    if not _ref_loaded:
        _ref = _load_ref()
        _ref_loaded = True
    return _ref


# ------------------------------------------------------------------ numpy wrappers


def quantize_q8_0(x, lib=None):
    """Row-wise Q8_0 quantization of x [..., K] (K % 32 == 0)."""
    lib = lib or oracle()
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows = x.reshape(-1, x.shape[-1])
    out = np.zeros((rows.shape[0], rows.shape[1] // QK), dtype=Q8)
    fn = lib.or_quantize_row_q8_0 if hasattr(lib, "or_quantize_row_q8_0") else lib.ei_quantize_row_q8_0
    for r in range(rows.shape[0]):
        fn(fptr(rows[r]), vptr(out[r]), rows.shape[1])
    return out.reshape(x.shape[:-1] + (x.shape[-1] // QK,))


def dequantize_q8_0(blocks):
    """Exact dequantization d*q of Q8_0 blocks [..., nb] -> [..., nb*32] float32."""
    d = np.frombuffer(np.ascontiguousarray(blocks["d"]).tobytes(), dtype=np.float16).astype(np.float32)
    d = d.reshape(blocks.shape)
    q = blocks["qs"].astype(np.float32)
    return (q * d[..., None]).reshape(blocks.shape[:-1] + (blocks.shape[-1] * QK,))


def host_libm(name, x):
    """The host libm's expf or tanhf of every element of x (float32)."""
    x = np.ascontiguousarray(x, np.float32)
    e, t = np.empty_like(x), np.empty_like(x)
    oracle().or_libm_eval(fptr(x), x.size, fptr(e), fptr(t))
    return {"expf": e, "tanhf": t}[name]


def gemm_q8_0(w, xq, threads=8):
    """y [n][m] from Q8_0 weights w [m][k/32] and Q8_0 activations xq [n][k/32]."""
    w = np.ascontiguousarray(w)
    xq = np.ascontiguousarray(xq)
    m, nb = w.shape
    n = xq.shape[0]
    y = np.zeros((n, m), dtype=np.float32)
    oracle().or_gemm_q8_0(vptr(w), vptr(xq), n, nb * QK, m, fptr(y), threads)
    return y


class OrLayer(C.Structure):
    _fields_ = [(n, _vp) for n in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_up", "ffn_gate", "ffn_down")] + [
        (n, _f)
        for n in ("attn_norm", "attn_q_norm", "attn_k_norm", "post_attention_norm", "ffn_norm", "post_ffw_norm")
    ] + [("rope_base", C.c_float), ("window", C.c_int32)]


class OrModel(C.Structure):
    _fields_ = [
        ("token_embd", _vp),
        ("output_norm", _f),
        ("dense_2", _vp),
        ("dense_3", _vp),
        ("n_layer", C.c_int32),
        ("eps", C.c_float),
        ("layers", OrLayer * 64),
    ]


def make_or_layer(L, rope_base, window):
    """L: dict of numpy arrays (Q8 matrices, float norms). Keeps references alive."""
    s = OrLayer()
    for n in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_up", "ffn_gate", "ffn_down"):
        setattr(s, n, vptr(L[n]))
    for n in ("attn_norm", "attn_q_norm", "attn_k_norm", "post_attention_norm", "ffn_norm", "post_ffw_norm"):
        setattr(s, n, fptr(L[n]))
    s.rope_base = rope_base
    s.window = window
    return s


def layer_forward(L, x, offsets, rope_base=10000.0, window=0, eps=1e-6, threads=8):
    """One encoder layer over a packed wave (in a copy of x)."""
    x = np.array(x, dtype=np.float32, copy=True)
    offsets = np.ascontiguousarray(offsets, dtype=np.uint64)
    batch = len(offsets) - 1
    pos = np.zeros(int(offsets[-1]), dtype=np.int32)
    for s in range(batch):
        pos[offsets[s]:offsets[s + 1]] = np.arange(offsets[s + 1] - offsets[s], dtype=np.int32)
    lay = make_or_layer(L, rope_base, window)
    oracle().or_layer_forward(C.byref(lay), eps, fptr(x), pos.ctypes.data_as(_i32), vptr(offsets), batch, threads)
    return x


def forward(model, ids, offsets, threads=8):
    """Whole packed-wave forward. model: dict with token_embd, output_norm,
    layers (list of dicts with rope_base/window), optional dense_2/dense_3."""
    m = OrModel()
    m.token_embd = vptr(model["token_embd"])
    m.output_norm = fptr(model["output_norm"])
    m.dense_2 = vptr(model["dense_2"]) if model.get("dense_2") is not None else None
    m.dense_3 = vptr(model["dense_3"]) if model.get("dense_3") is not None else None
    m.n_layer = len(model["layers"])
    m.eps = model.get("eps", 1e-6)
    for i, L in enumerate(model["layers"]):
        m.layers[i] = make_or_layer(L, L["rope_base"], L["window"])
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    offsets = np.ascontiguousarray(offsets, dtype=np.uint64)
    batch = len(offsets) - 1
    out = np.zeros((batch, N_EMBD), dtype=np.float32)
    rc = oracle().or_forward(C.byref(m), ids.ctypes.data_as(_i32), vptr(offsets), batch, fptr(out), threads)
    if rc != 0:
        raise ValueError("oracle rejected the wave")
    return out
