"""Host-side checks of libeg2hip.so that need no GPU: exported symbols,
argument validation, RoPE tables, Q8_0 repacking and the GGUF writer/reader."""
import ctypes as C
import hashlib
import os
import re

import numpy as np
import pytest

import gguf_py
from oracle_lib import Q8, dequantize_q8_0, fptr, oracle, quantize_q8_0

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in ("gemma2_kfd.h", "eg2_hip.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b((?:ei|eg2)_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol(eg2):
    lib = eg2.lib()
    names = declared_functions()
    assert {"ei_gemma2_kfd_create", "ei_gemma2_kfd_free", "ei_gemma2_kfd_batch", "eg2_hip_gemm_q8",
            "eg2_hip_attention"} <= names
    for n in names:
        assert hasattr(lib, n), n
    assert names <= set(eg2.SIGNATURES), names - set(eg2.SIGNATURES)


def test_operator_abi_header_matches_reference_records():
    """include/abi.h keeps the nine records of kernels/abi.h:3-11 field for field."""
    text = open(os.path.join(ROOT, "include", "abi.h")).read()
    want = {
        "EgGather": "float *out; const void *weight; const int *ids; unsigned n;",
        "EgMM": "float *out; const float *x; const void *weight; unsigned n, k, m, type;",
        "EgNorm": "float *out; const float *x; const float *weight; unsigned rows, d; float scale;",
        "EgRope": "float *x; const float *table; unsigned n, heads, d;",
        "EgAttention": "float *out; const float *q, *k, *v; const unsigned *bounds; unsigned n, window;",
        "EgElement": "float *out; const float *x, *other; unsigned n, mode, layer; float scale;",
        "EgPool": "float *out; const float *x; const unsigned *offsets; unsigned batch;",
        "EgNormResidual": "float *out; const float *x, *weight; unsigned rows, d; float scale;",
        "EgNormRope": "float *x; const float *weight, *table; unsigned rows, d, heads;",
    }
    for name, fields in want.items():
        assert f"typedef struct {{ {fields} }} {name};" in text, name


def test_ops_reject_bad_arguments_without_launching(eg2):
    lib = eg2.lib()
    inval = 1  # hipErrorInvalidValue
    p = C.c_void_p(16)
    assert lib.eg2_hip_gemm_q8(p, p, p, p, p, 4, 4, 33, 4, None) == inval  # k % 32
    assert lib.eg2_hip_gemm_q8(p, p, p, p, p, 4, 8, 32, 4, None) == inval  # ldy < m
    assert lib.eg2_hip_gemm_q8(None, p, p, p, p, 4, 4, 32, 4, None) == inval
    assert lib.eg2_hip_attention(p, p, p, p, p, 0, 0, 32, p, p, None) == inval  # grid 0
    assert lib.eg2_hip_attention(p, p, p, p, p, 4, 99999, 32, p, p, None) == inval
    assert lib.eg2_hip_attention(p, p, p, None, p, 4, 0, 32, p, p, None) == inval
    assert lib.eg2_hip_quantize_rows(p, 96, p, p, 1, None) == inval  # k % 64
    assert lib.eg2_hip_l2_prefix(p, 768, 769, 1, None) == inval
    assert lib.eg2_hip_l2_prefix(p, 768, 100, 1, None) == inval
    assert lib.eg2_hip_pool_l2(p, p, p, 0, None) == inval


def test_attention_tiles_cover_each_sequence(eg2):
    offs = [0, 1, 33, 97, 98, 200]
    arr = (C.c_size_t * len(offs))(*offs)
    tiles = np.zeros(4 * 200, np.uint32)
    n = eg2.lib().eg2_attention_tiles(arr, len(offs) - 1, tiles.ctypes.data)
    t = tiles[:4 * n].reshape(n, 4)
    covered = np.zeros(200, int)
    for q0, q1, lo, hi in t:
        assert lo <= q0 < q1 <= hi and q1 - q0 <= 32 and (q0 - lo) % 32 == 0
        assert [lo, hi] in [[offs[s], offs[s + 1]] for s in range(len(offs) - 1)]
        covered[q0:q1] += 1
    assert (covered == 1).all()
    assert n == sum((offs[s + 1] - offs[s] + 31) // 32 for s in range(len(offs) - 1))


@pytest.mark.parametrize("base", [10000.0, 1000000.0])
def test_rope_table_matches_oracle(eg2, base):
    t = eg2.rope_table(base)
    o = oracle()
    c = np.zeros(128, np.float32)
    s = np.zeros(128, np.float32)
    for p in list(range(0, 2048, 7)) + [2047]:
        o.or_rope_cos_sin(p, base, fptr(c), fptr(s))
        assert np.array_equal(t[p, :128], c), p
        assert np.array_equal(t[p, 128:], s), p


def test_q8_split_is_the_exact_decode(eg2):
    rng = np.random.default_rng(0)
    blocks = quantize_q8_0((rng.standard_normal((10, 96)) * 10.0 ** rng.uniform(-6, 2, (10, 1))).astype(np.float32))
    blocks[0, 0]["qs"][:4] = [-128, 127, 0, -1]
    q, d = eg2.q8_split(blocks.view(np.uint8), 10, 96)
    assert q.dtype == np.float16
    assert np.array_equal(q.reshape(10, 3, 32).astype(np.int32), blocks["qs"].astype(np.int32))
    assert np.array_equal(d, blocks["d"].view(np.float16).astype(np.float32))
    deq = (q.reshape(10, 3, 32).astype(np.float32) * d[:, :, None]).reshape(10, 96)
    assert np.array_equal(deq, dequantize_q8_0(blocks))


@pytest.fixture(scope="module")
def small_gguf(eg2, tmp_path_factory):
    path = str(tmp_path_factory.mktemp("gguf") / "m.gguf")
    eg2.synth_gguf(path, seed=3, n_layer=2, dense_head=True, threads=4, sliding_window=512, rope_base_full=1e6)
    return path


def test_synthetic_gguf_reads_back_identically(eg2, small_gguf):
    kvs, tensors = gguf_py.read(small_gguf)
    assert kvs["general.architecture"] == "gemma-embedding"
    assert kvs["gemma-embedding.block_count"] == 2
    g = eg2.Gguf(small_gguf)
    try:
        assert g.g.version == 3 and g.g.n_tensors == len(tensors)
        names = {}
        for i in range(g.g.n_tensors):
            t = g.g.tensors[i]
            name = C.string_at(t.name.str, t.name.len).decode()
            names[name] = t
        assert set(names) == set(tensors)
        for name, (ty, ne, arr) in tensors.items():
            t = names[name]
            assert t.type == ty and list(t.ne[: t.n_dims]) == ne
            raw = np.ctypeslib.as_array((C.c_uint8 * t.n_bytes).from_address(t.data))
            assert np.array_equal(raw, arr.view(np.uint8).reshape(-1)), name
        kv = {C.string_at(g.g.kv[i].key.str, g.g.kv[i].key.len).decode(): g.g.kv[i] for i in range(g.g.n_kv)}
        assert kv["gemma-embedding.rope.freq_base"].v.f64 == 1e6
        assert kv["gemma-embedding.attention.sliding_window"].v.u64 == 512
    finally:
        g.close()


def test_synthetic_weights_follow_the_stated_distribution(small_gguf):
    kvs, t = gguf_py.read(small_gguf)
    w = dequantize_q8_0(t["blk.0.ffn_up.weight"][2])
    assert w.shape == (1152, 768)
    assert abs(w.std() - 0.02) < 0.001 and abs(w.mean()) < 0.001
    # Re-quantizing the dequantized weights reproduces the stored blocks: they
    # were written by the reference quantizer rules.
    again = quantize_q8_0(w.astype(np.float32))
    assert np.array_equal(again.view(np.uint8), t["blk.0.ffn_up.weight"][2].view(np.uint8))
    n = t["blk.1.post_ffw_norm.weight"][2]
    assert abs(n.mean() - 1.0) < 0.02 and abs(n.std() - 0.1) < 0.02


def test_synthetic_gguf_independent_of_thread_count(eg2, tmp_path):
    digests = []
    for threads in (1, 5):
        p = str(tmp_path / f"m{threads}.gguf")
        eg2.synth_gguf(p, seed=9, n_layer=1, dense_head=False, threads=threads)
        digests.append(hashlib.sha256(open(p, "rb").read()).hexdigest())
    assert digests[0] == digests[1]


def test_gguf_reader_rejects_malformed_files(eg2, tmp_path):
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUF\x02\x00\x00\x00" + b"\x00" * 16)
    with pytest.raises(eg2.HipError, match="version"):
        eg2.Gguf(str(bad))
    bad.write_bytes(b"NOPE" + b"\x00" * 40)
    with pytest.raises(eg2.HipError, match="not a GGUF"):
        eg2.Gguf(str(bad))
    with pytest.raises(eg2.HipError, match="cannot open"):
        eg2.Gguf(str(tmp_path / "missing.gguf"))


def test_executor_create_reports_missing_device(eg2, small_gguf):
    err = C.create_string_buffer(256)
    if eg2.lib().eg2_hip_device_check(err, 256) == 0:
        pytest.skip("a gfx950 device is present; covered by the GPU tests")
    with pytest.raises(eg2.HipError, match=r"^HIP: supported HIP device not found"):
        eg2.Encoder(small_gguf)
