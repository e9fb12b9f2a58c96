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
    for h in ("gemma2_kfd.h", "eg2_hip.h", "eg2_ops.h", "eg2_stream.h"):
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


def test_lane_query_rejects_an_empty_context(eg2):
    err = C.create_string_buffer(256)
    assert eg2.lib().eg2_kfd_lane_ready(None, 0, err, 256) == -1
    assert b"empty context" in err.value


def test_ops_reject_bad_arguments_without_launching(eg2):
    lib = eg2.lib()
    inval = 1  # hipErrorInvalidValue
    p = C.c_void_p(16)
    assert lib.eg2_hip_gemm_q8(p, p, 4, p, p, 4, p, 4, 4, 33, 4, None) == inval  # k % 32
    assert lib.eg2_hip_gemm_q8(p, p, 4, p, p, 8, p, 4, 8, 32, 4, None) == inval  # ldy < m
    assert lib.eg2_hip_gemm_q8(p, p, 3, p, p, 4, p, 4, 4, 32, 4, None) == inval  # ldx < n
    assert lib.eg2_hip_gemm_q8(p, p, 4, p, p, 3, p, 4, 4, 32, 4, None) == inval  # ldw < m
    assert lib.eg2_hip_gemm_q8(p, p, 4, p, p, 4, p, 4, 4, 1 << 25, 4, None) == inval  # k above 2^24
    assert lib.eg2_hip_gemm_q8(None, p, 4, p, p, 4, p, 4, 4, 32, 4, None) == inval
    # scale arrays of 4 GiB or more: (k/32) ldx 4 = 2^19 * 8192 * 4 bytes
    assert lib.eg2_hip_gemm_q8(p, p, 8192, p, p, 4, p, 4, 4, 1 << 24, 4, None) == inval
    assert lib.eg2_hip_gemm_q8(p, p, 4, p, p, 8192, p, 4, 4, 1 << 24, 4, None) == inval
    # gemm_q8_qkv_rope(xq, xd, ldx, wq, wd, ldw, n, k, q_w, k_w, rope, pos, eps, out)
    f = C.c_float(1e-6)
    assert lib.eg2_hip_gemm_q8_qkv_rope(p, p, 4, p, p, 1280, 4, 48, p, p, p, p, f, p, None) == inval  # k % 32
    assert lib.eg2_hip_gemm_q8_qkv_rope(p, p, 4, p, p, 1279, 4, 32, p, p, p, p, f, p, None) == inval  # ldw
    assert lib.eg2_hip_gemm_q8_qkv_rope(p, p, 3, p, p, 1280, 4, 32, p, p, p, p, f, p, None) == inval  # ldx < n
    assert lib.eg2_hip_gemm_q8_qkv_rope(p, p, 4, p, p, 1280, 4, 32, p, p, p, None, f, p, None) == inval
    assert lib.eg2_hip_gemm_q8_qkv_rope(p, p, 4, p, p, 1280, 4, 32, p, p, p, p, f, None, None) == inval
    assert lib.eg2_hip_gemm_q8_qkv_rope(p, p, 8192, p, p, 1280, 4, 1 << 24, p, p, p, p, f, p, None) == inval
    # gemm_q8_geglu(xq, xd, ldx, wq, wd, ldw, gq, gd, ldg, n, ff, k)
    assert lib.eg2_hip_gemm_q8_geglu(p, p, 4, p, p, 96, p, p, 4, 4, 48, 32, None) == inval  # ff % 32
    assert lib.eg2_hip_gemm_q8_geglu(p, p, 4, p, p, 64, p, p, 4, 4, 32, 48, None) == inval  # k % 32
    assert lib.eg2_hip_gemm_q8_geglu(p, p, 4, p, p, 63, p, p, 4, 4, 32, 32, None) == inval  # ldw < 2 ff
    assert lib.eg2_hip_gemm_q8_geglu(p, p, 3, p, p, 64, p, p, 4, 4, 32, 32, None) == inval  # ldx < n
    assert lib.eg2_hip_gemm_q8_geglu(p, p, 4, p, p, 64, p, p, 3, 4, 32, 32, None) == inval  # ldg < n
    assert lib.eg2_hip_gemm_q8_geglu(p, p, 4, p, p, 64, p, None, 4, 4, 32, 32, None) == inval
    assert lib.eg2_hip_gemm_q8_geglu(p, p, 4, p, p, 64, p, p, 4, 0, 32, 32, None) == inval  # n = 0
    assert lib.eg2_hip_gemm_q8_geglu(p, p, 4, p, p, 8192, p, p, 4, 4, 32, 1 << 24, None) == inval  # w scales 16 GiB
    # attention(qkv, items, item_count, grid, tok, window, rows, longest, scores, cq, cd)
    assert lib.eg2_hip_attention(p, p, p, 0, p, 0, 32, 0, p, p, p, None) == inval  # grid 0
    assert lib.eg2_hip_attention(p, p, p, 64, p, 99999, 32, 0, p, p, p, None) == inval  # window
    assert lib.eg2_hip_attention(p, p, p, 64, None, 0, 32, 0, p, p, p, None) == inval
    assert lib.eg2_hip_attention(p, p, p, 64, p, 0, 30, 0, p, p, p, None) == inval  # rows % 4
    assert lib.eg2_hip_attention(p, p, p, 64, p, 0, 32, 0, None, p, p, None) == inval  # no scratch
    assert lib.eg2_hip_attention(p, p, p, 64, p, 0, 32, 33, p, p, p, None) == inval  # longest > rows
    # the three stages of attention
    assert lib.eg2_hip_attention_scores(p, p, p, 0, 0, 32, p, None) == inval  # grid 0
    assert lib.eg2_hip_attention_scores(p, p, p, 64, 0, 30, p, None) == inval  # rows % 4
    assert lib.eg2_hip_attention_scores(p, p, p, 64, 0, 32, None, None) == inval  # no scratch
    assert lib.eg2_hip_attention_softmax(None, 0, 32, 0, p, None) == inval
    assert lib.eg2_hip_attention_softmax(p, 0, 32, 33, p, None) == inval  # longest > rows
    assert lib.eg2_hip_attention_softmax(p, 99999, 32, 0, p, None) == inval  # window
    assert lib.eg2_hip_attention_context(p, p, p, 64, 0, 32, p, None, p, None) == inval
    assert lib.eg2_hip_attention_context(p, p, p, 64, 0, 30, p, p, p, None) == inval  # rows % 4
    assert lib.eg2_hip_qk_norm_rope(p, p, p, p, p, f, None, 4, None) == inval
    assert lib.eg2_hip_qk_norm_rope(p, p, p, p, p, f, p, 0, None) == inval
    assert lib.eg2_hip_libm_eval(p, 0, p, p, None) == inval
    assert lib.eg2_hip_quantize_rows(p, 96, p, p, 1, None) == inval  # k % 64
    assert lib.eg2_hip_l2_prefix(p, 768, 769, 1, None) == inval
    assert lib.eg2_hip_l2_prefix(p, 768, 100, 1, None) == inval
    assert lib.eg2_hip_pool_l2(p, p, p, 0, None) == inval
    assert lib.eg2_hip_pool_mean(p, p, p, 0, None) == inval
    assert lib.eg2_hip_pool_mean(p, p, p, 65536, None) == inval


def test_attention_plan_covers_each_sequence(eg2):
    """Every (pair, key) of each sequence (pair = 3 (token - start) + head)
    is covered by exactly one score item (32-key blocks from the sequence
    start times 32-pair blocks), every pair by exactly one context item
    (32-pair blocks), the score items coming first; the 1/sum area takes
    ceil4(3 rows) floats, then each sequence's scores 3 n ceil4(n) floats
    after the previous ones; every token's record names its sequence and
    that first score index."""
    offs = [0, 1, 33, 97, 98, 200, 600, 1100, 3150]
    items, tok, score_floats, n_score = eg2.attention_plan(offs)
    seqs = [(offs[s], offs[s + 1]) for s in range(len(offs) - 1)]
    c4 = lambda n: (n + 3) // 4 * 4  # noqa: E731
    base = np.concatenate([[c4(3 * offs[-1])],
                           c4(3 * offs[-1]) + np.cumsum([3 * (b - a) * c4(b - a) for a, b in seqs])])
    assert score_floats == base[-1]
    covered = {s: np.zeros((3 * (hi - lo), hi - lo), int) for s, (lo, hi) in enumerate(seqs)}
    ctx = {s: np.zeros(3 * (hi - lo), int) for s, (lo, hi) in enumerate(seqs)}
    for i, (lo, hi, f2, f3, f4, f5, f6, f7) in enumerate(items.astype(np.int64)):
        s = seqs.index((lo, hi))
        n = hi - lo
        if i < n_score:
            k0, p0, p1, sb = f2, f3, f4, f5
            assert sb == base[s] and f6 == f7 == 0
            assert lo <= k0 < hi and (k0 - lo) % 32 == 0
            assert 0 <= p0 < p1 <= 3 * n and p0 % 32 == 0 and p1 == min(3 * n, p0 + 32)
            covered[s][p0:p1, k0 - lo:min(hi, k0 + 32) - lo] += 1
        else:
            p0, p1, sb = f2, f3, f4
            assert sb == base[s] and f5 == items[n_score][5] and f6 == f7 == 0
            assert p0 % 32 == 0 and p1 == min(3 * n, p0 + 32)
            ctx[s][p0:p1] += 1
    for s in covered:
        assert (covered[s] == 1).all(), s
        assert (ctx[s] == 1).all(), s
    for s, (lo, hi) in enumerate(seqs):
        assert (tok[lo:hi] == [lo, hi, base[s], 0]).all()


def test_attention_plan_context_order_follows_balance(eg2):
    """The context items carry the context kernel's unit order: XCD-contiguous
    eighths (1) for packings whose eighths of units cost alike (equal
    sequences, the 16 x 128 wave, also with a short padding sequence after
    it), the plain stride (0) for mixed ones, whose contiguous eighths would
    give some XCDs all the long sequences."""
    def flag(offs):
        items, _, _, n_score = eg2.attention_plan(offs)
        f = set(items[n_score:, 5].tolist())
        assert len(f) == 1
        return f.pop()

    assert flag(list(range(0, 2049, 128))) == 1
    assert flag(list(range(0, 2049, 512))) == 1
    assert flag(list(range(0, 1601, 100)) + [1632]) == 1
    assert flag([0, 105, 128, 137, 145, 364, 695, 788, 943, 1014, 1377, 1598, 1606, 1869, 1878, 2033, 2048]) == 0
    assert flag([0, 2048]) == 1
    assert flag([0, 1]) == 0  # 4 units: fewer than the XCDs


def test_attention_plan_checks_capacity_before_writing(eg2):
    """A plan that does not fit the given capacity is rejected with nothing
    written (the counts still report the need)."""
    import ctypes as C

    offs = [0, 700, 1500]
    items0, _, need_scores, n_score = eg2.attention_plan(offs)
    need_items = len(items0)
    assert need_scores == 4500 + 3 * (700 * 700 + 800 * 800)
    arr = (C.c_size_t * 3)(*offs)
    items = np.full((need_items, 8), 7, np.uint32)
    tok = np.full((1500, 4), 7, np.uint32)
    counts = (C.c_size_t * 3)()
    for cap_items, cap_scores in ((need_items - 1, 1 << 30), (need_items, need_scores - 1)):
        rc = eg2.lib().eg2_attention_plan(arr, 2, cap_items, cap_scores, items.ctypes.data, tok.ctypes.data, counts)
        assert rc == -1 and list(counts) == [need_items, need_scores, n_score]
        assert (items == 7).all() and (tok == 7).all()


def test_attention_plan_refuses_scores_past_32_bits(eg2):
    """The plan's records hold 32-bit score indices: a packing whose score
    floats pass 2^32 (one sequence of 40,000 tokens: 3 n ceil4(n) = 4.8e9)
    is refused even with room to spare, with nothing written."""
    import ctypes as C

    n = 40000
    arr = (C.c_size_t * 2)(0, n)
    items = np.full((8, 8), 7, np.uint32)
    tok = np.full((8, 4), 7, np.uint32)
    counts = (C.c_size_t * 3)()
    rc = eg2.lib().eg2_attention_plan(arr, 1, 1 << 40, 1 << 40, items.ctypes.data, tok.ctypes.data, counts)
    assert rc == -1 and counts[1] == 3 * n + 3 * n * n and counts[1] > 2 ** 32
    assert (items == 7).all() and (tok == 7).all()


def test_attention_capacity_bounds_every_packing(eg2):
    """The executor sizes its plan with eg2_attention_capacity(2080, 2049)
    (a 2048-token wave plus a padding sequence of up to 31 rows): no packing
    may exceed it. Every packing of equal sequences (the per-sequence
    rounding of blocks is worst there) and every remainder, each followed by
    its padding sequence."""
    cap = eg2.attention_capacity(2080, 2049)
    worst = [0, 0]
    for L in range(1, 2049):
        for total in (2048, 2048 - L // 2, 2017):
            lens = [L] * (total // L) + ([total % L] if total % L else [])
            n = sum(lens)
            pad = (-n) % 32
            offs = np.concatenate([[0], np.cumsum(lens + ([pad] if pad else []))])
            items, _, score_floats, _ = eg2.attention_plan(offs)
            got = [len(items), score_floats]
            worst = [max(a, b) for a, b in zip(worst, got)]
            assert all(g <= c for g, c in zip(got, cap)), (L, total, got, cap)
    print("worst", worst, "capacity", cap)


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


def tile_offset(r, e, k):
    """Byte offset of value e of row r in a row-tile buffer, written out from
    the layout's definition: [rows/32][k/32][2][32][16] int8."""
    return ((((r // 32) * (k // 32) + e // 32) * 2 + (e // 16) % 2) * 32 + r % 32) * 16 + e % 16


def test_q8_row_tiles_layout_and_round_trip(eg2):
    rng = np.random.default_rng(0)
    for rows, k in [(1, 32), (45, 96), (64, 768), (33, 1152)]:
        q = rng.integers(-128, 128, (rows, k)).astype(np.int8)
        tiles = eg2.q8_pack_rows(q)
        assert tiles.size == eg2.q8_tile_bytes(rows, k) == -(-rows // 32) * (k // 32) * 1024
        r, e = np.meshgrid(np.arange(rows), np.arange(k), indexing="ij")
        assert np.array_equal(tiles[tile_offset(r, e, k)], q)
        covered = np.zeros(tiles.size, bool)
        covered[tile_offset(r, e, k)] = True
        assert not tiles[~covered].any()  # padding rows are zero
        assert np.array_equal(eg2.q8_unpack_rows(tiles, rows, k), q)


def test_q8_weight_tiles_are_the_exact_decode(eg2):
    """Weights: int8 values in row tiles and the exact float value of each
    fp16 block scale, transposed [k/32][rows rounded up to 32] (zero past
    the matrix); value * scale is the reference dequantization."""
    rng = np.random.default_rng(1)
    rows, k = 45, 96
    blocks = quantize_q8_0((rng.standard_normal((rows, k)) * 10.0 ** rng.uniform(-6, 2, (rows, 1))).astype(np.float32))
    blocks[0, 0]["qs"][:4] = [-128, 127, 0, -1]
    wq, wd = eg2.q8_weight_tiles(blocks.view(np.uint8), rows, k)
    assert wd.shape == (3, 64)
    q = eg2.q8_unpack_rows(wq, rows, k)
    assert np.array_equal(q.reshape(rows, 3, 32), blocks["qs"])
    assert np.array_equal(wd[:, :rows].T, blocks["d"].view(np.float16).astype(np.float32))
    assert not wd[:, rows:].any()
    assert not eg2.q8_unpack_rows(wq, 64, k)[rows:].any()
    deq = (q.reshape(rows, 3, 32).astype(np.float32) * wd[:, :rows].T[:, :, None]).reshape(rows, k)
    assert np.array_equal(deq, dequantize_q8_0(blocks))


def test_q8_geglu_weight_tiles_interleave_gate_and_up(eg2):
    """The fused gate|up + GeGLU operands are the plain weight tiles of
    [gate 0-31, up 0-31, gate 32-63, up 32-63, ...]."""
    rng = np.random.default_rng(2)
    ff, k = 96, 64
    gate = quantize_q8_0(rng.standard_normal((ff, k)).astype(np.float32))
    up = quantize_q8_0((rng.standard_normal((ff, k)) * 3).astype(np.float32))
    wq, wd = eg2.q8_geglu_weight_tiles(gate.view(np.uint8), up.view(np.uint8), ff, k)
    order = np.concatenate([np.concatenate([gate[32 * j:32 * j + 32], up[32 * j:32 * j + 32]]) for j in range(ff // 32)])
    rq, rd = eg2.q8_weight_tiles(order.view(np.uint8), 2 * ff, k)
    assert np.array_equal(wq, rq) and np.array_equal(wd, rd)
    q = eg2.q8_unpack_rows(wq, 2 * ff, k).reshape(ff // 32, 2, 32, k)
    assert np.array_equal(q[1, 0], gate["qs"][32:64].reshape(32, k))
    assert np.array_equal(q[2, 1], up["qs"][64:96].reshape(32, k))
    with pytest.raises(ValueError):
        eg2.q8_geglu_weight_tiles(gate[:40].view(np.uint8), up[:40].view(np.uint8), 40, k)


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


def _tensor(g, name):
    for i in range(g.g.n_tensors):
        t = g.g.tensors[i]
        if C.string_at(t.name.str, t.name.len).decode() == name:
            return t
    raise KeyError(name)


@pytest.mark.parametrize("name,change,msg", [
    # n_dims 3 with ne[2] = 0: a zero byte count that passes the reader's
    # bounds check but would make the embedding gather read past the upload.
    ("token_embd.weight", dict(n_dims=3, ne2=0, n_bytes=0), "unexpected shape: token_embd.weight"),
    ("output_norm.weight", dict(n_bytes=256), "unexpected byte count: output_norm.weight"),
    ("blk.0.attn_norm.weight", dict(n_dims=3, ne2=2, n_bytes=768 * 4 * 2), "unexpected shape: blk.0.attn_norm"),
    ("blk.1.attn_q_norm.weight", dict(ne0=128, n_bytes=512), "unexpected shape: blk.1.attn_q_norm"),
    ("blk.1.ffn_down.weight", dict(type=0), "unexpected type: blk.1.ffn_down.weight"),
    ("blk.0.attn_q.weight", dict(n_bytes=768 * 24 * 34 - 34), "unexpected byte count: blk.0.attn_q.weight"),
    ("blk.0.attn_k.weight", dict(ne3=0), "unexpected shape: blk.0.attn_k.weight"),
    ("blk.1.ffn_up.weight", dict(rename=True), "missing tensor: blk.1.ffn_up.weight"),
    ("dense_3.weight", dict(rename=True), "dense_2/dense_3 must be both present or absent"),
])
def test_model_validation_rejects_malformed_tensor_records(eg2, small_gguf, name, change, msg):
    """Every tensor record the executor reads is checked for type, shape and
    exact byte count on the host, before create makes any device call."""
    g = eg2.Gguf(small_gguf)
    try:
        assert eg2.validate_gguf(g) is None
        t = _tensor(g, name)
        if change.get("rename"):
            t.name.len = 3  # a different name
        for f in ("n_dims", "type", "n_bytes"):
            if f in change:
                setattr(t, f, change[f])
        for i in range(4):
            if f"ne{i}" in change:
                t.ne[i] = change[f"ne{i}"]
        got = eg2.validate_gguf(g)
        assert got is not None and got.startswith("HIP: ") and msg in got, got
        # create reports the same rejection: the checks run before the
        # device is touched (here, before finding there is none).
        err = C.create_string_buffer(512)
        assert not eg2.lib().ei_gemma2_kfd_create(C.byref(g.g), err, 512)
        assert msg in err.value.decode()
    finally:
        g.close()


REFERENCE_OPERATORS = {"eg2_saxpy", "eg2_gather", "eg2_mm", "eg2_mm64", "eg2_mm64x64", "eg2_mmstep8", "eg2_norm",
                       "eg2_rope", "eg2_attention256", "eg2_attention512", "eg2_element", "eg2_pool",
                       "eg2_norm_residual", "eg2_norm_rope"}  # kernels/eg2.c


def test_operator_names_cover_the_reference_set(eg2):
    lib = eg2.lib()
    names = {lib.eg2_op_name(i).decode() for i in range(lib.eg2_op_count())}
    assert names == REFERENCE_OPERATORS | {"eg2_gather768", "eg2_attention256x3"}
    assert lib.eg2_op_name(lib.eg2_op_count()) is None


def test_operator_records_match_the_c_layout(tmp_path, eg2):
    """ctypes records == the C layout of include/abi.h (size and offsets)."""
    import subprocess

    recs = ["EgGather", "EgMM", "EgNorm", "EgRope", "EgAttention", "EgElement", "EgPool", "EgNormResidual",
            "EgNormRope", "EgSaxpy"]
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "eg2_ops.h"', "int main(void) {"]
    for r in recs:
        lines.append(f'  printf("{r} %zu\\n", sizeof({r}));')
        for f, _ in getattr(eg2, r)._fields_:
            lines.append(f'  printf("{r}.{f} %zu\\n", offsetof({r}, {f}));')
    lines.append("  return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    out = dict(line.split() for line in subprocess.run([str(exe)], check=True, capture_output=True,
                                                        text=True).stdout.splitlines())
    for r in recs:
        cls = getattr(eg2, r)
        assert int(out[r]) == C.sizeof(cls), r
        for f, _ in cls._fields_:
            assert int(out[f"{r}.{f}"]) == getattr(cls, f).offset, (r, f)


def test_operator_launch_rejects_bad_arguments_without_launching(eg2):
    """Every case fails validation before any launch (no device needed)."""
    lib = eg2.lib()
    p = 16  # a non-null pointer value; nothing is launched

    def launch(name, rec, gx=1, gy=1, block=256, size=None):
        return lib.eg2_op_launch(name.encode(), C.byref(rec), C.sizeof(rec) if size is None else size, gx, gy,
                                 block, None)

    inval = 1
    mm = eg2.EgMM(p, p, p, 4, 32, 4, 8)
    assert launch("eg2_nope", mm) == inval
    assert launch("eg2_mm", mm, size=C.sizeof(mm) - 4) == inval
    assert launch("eg2_mm", mm, gx=0) == inval
    assert launch("eg2_mm", mm, block=128) == inval
    assert launch("eg2_mm", eg2.EgMM(p, p, p, 4, 32, 4, 2)) == inval  # GGML type 2 is not supported
    assert launch("eg2_mm", eg2.EgMM(None, p, p, 4, 32, 4, 8)) == inval
    assert launch("eg2_norm", eg2.EgNorm(p, p, None, 1, 16, 1.0), block=256) == inval
    assert launch("eg2_norm", eg2.EgNorm(p, p, None, 1, 0, 1.0), block=64) == inval
    assert launch("eg2_rope", eg2.EgRope(p, p, 1, 1, 7)) == inval
    assert launch("eg2_norm_rope", eg2.EgNormRope(p, p, p, 1, 256, 0), block=64) == inval
    assert launch("eg2_element", eg2.EgElement(p, p, p, 8, 3, 0, 1.0)) == inval
    assert launch("eg2_attention256", eg2.EgAttention(p, p, p, p, None, 1, 0), block=64) == inval
    assert launch("eg2_pool", eg2.EgPool(p, p, None, 1)) == inval
    assert launch("eg2_saxpy", eg2.EgSaxpy(None, p, 1.0, 4)) == inval
    assert lib.eg2_op_launch(None, C.byref(mm), C.sizeof(mm), 1, 1, 256, None) == inval


def elf_symbols(path):
    """Names in the .symtab of a 64-bit little-endian ELF file."""
    import struct

    data = open(path, "rb").read()
    assert data[:4] == b"\x7fELF" and data[4] == 2 and data[5] == 1
    shoff, = struct.unpack_from("<Q", data, 0x28)
    shentsize, shnum = struct.unpack_from("<HH", data, 0x3A)
    sections = [struct.unpack_from("<IIQQQQIIQQ", data, shoff + i * shentsize) for i in range(shnum)]
    names = set()
    for sh in sections:
        if sh[1] != 2:  # SHT_SYMTAB
            continue
        strtab = sections[sh[6]]
        for off in range(sh[4], sh[4] + sh[5], sh[9]):
            name_off, = struct.unpack_from("<I", data, off)
            s = data[strtab[4] + name_off:data.index(b"\0", strtab[4] + name_off)]
            names.add(s.decode())
    return names


def test_code_object_exports_the_operator_kernels(eg2):
    """The stand-alone gfx950 code object carries NAME and NAME.kd for every
    operator, as a by-name loader expects (src/gemma2_kfd.cpp:106-110)."""
    co = os.path.join(ROOT, "embeddinggemma2-amdkfd_amd", "eg2_ops_gfx950.co")
    syms = elf_symbols(co)
    lib = eg2.lib()
    for i in range(lib.eg2_op_count()):
        name = lib.eg2_op_name(i).decode()
        assert name in syms and name + ".kd" in syms, name


@pytest.mark.parametrize("source,dma", [("kernels_attn.hip", True), ("kernels_gemm.hip", False)])
def test_dma_is_the_only_m0_user(tmp_path, source, dma):
    """The attention kernels set M0 in inline asm for their LDS DMA and
    declare it clobbered; that is sound only while no compiler-generated
    instruction in those kernels reads M0. Compiles the source for gfx950
    with the library's flags and checks that every mention of m0 in the ISA
    is the asm's own write (a compiler update or a new M0 user fails here).
    The projection GEMMs load their operands into registers and use no M0
    at all."""
    import shutil
    import subprocess

    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    if not shutil.which(hipcc):
        pytest.skip("hipcc not available")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    pkg = os.path.join(root, "embeddinggemma2-amdkfd_amd")
    out = tmp_path / "gemm.s"
    cmd = [hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
           "-fhip-fp32-correctly-rounded-divide-sqrt", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-mllvm", "-amdgpu-mfma-vgpr-form", "-I" + os.path.join(root, "include"), "-I" + os.path.join(pkg, "csrc"),
           "--cuda-device-only", "-S", os.path.join(pkg, "csrc", source), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    writes = others = 0
    for line in out.read_text().splitlines():
        code = line.split(";")[0]
        if not re.search(r"\bm0\b", code):
            continue
        if re.match(r"\s*s_mov_b32 m0, s\d+\s*$", code):
            writes += 1
        else:
            others += 1
    assert (writes > 0) == dma and others == 0, (writes, others)
