"""Tokenizer parity (include/eg2_tokenizer.h) with the reference's
tokenizer.c, bit for bit.

tests/golden/tokenizer_vectors.npz holds three synthetic vocabularies (two
SentencePiece-style ones with different BOS/EOS/space-prefix flags and one
with ranked merge rules, the reference's embeddinggemma2 mode), 401 seeded
texts (specials inside and overlapping, byte fallback, invalid UTF-8, the vocabularies' own words,
newline runs, tabs, multi-byte characters, a long text) and the ids the
compiled reference gives each text under every (add_special,
parse_special) pair. Each vocabulary is written back into a GGUF file with
the same key-value writer the fixture script used and read by this build's
own GGUF reader."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import gguf_py  # noqa: E402

GOLDEN = os.path.join(ROOT, "tests", "golden", "tokenizer_vectors.npz")
COMBOS = [(1, 0), (1, 1), (0, 0), (0, 1)]


def unblob(data, offs):
    b = data.tobytes()
    return [b[offs[i]:offs[i + 1]] for i in range(len(offs) - 1)]


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN)


def make_tokenizer(eg2, g, name, path):
    make_tokenizer_file(g, name, path)
    return eg2.Tokenizer(path)


def make_tokenizer_file(g, name, path):
    """Writes vocabulary `name` of the fixture as a GGUF file of tokenizer keys."""
    bos, eos, add_bos, add_eos, prefix = (int(x) for x in g[f"{name}_flags"])
    kvs = [("tokenizer.ggml.model", "str", "llama"),
           ("tokenizer.ggml.tokens", "arr_str", unblob(g[f"{name}_tokens"], g[f"{name}_token_offsets"])),
           ("tokenizer.ggml.scores", "arr_f32", g[f"{name}_scores"]),
           ("tokenizer.ggml.token_type", "arr_i32", g[f"{name}_types"]),
           ("tokenizer.ggml.bos_token_id", "u32", bos), ("tokenizer.ggml.eos_token_id", "u32", eos),
           ("tokenizer.ggml.add_bos_token", "bool", add_bos), ("tokenizer.ggml.add_eos_token", "bool", add_eos),
           ("tokenizer.ggml.add_space_prefix", "bool", prefix)]
    merges = unblob(g[f"{name}_merges"], g[f"{name}_merge_offsets"])
    if merges:
        kvs.append(("tokenizer.ggml.merges", "arr_str", merges))
    gguf_py.write_kv(path, kvs)


@pytest.mark.parametrize("name", ["spm", "spm_eos", "ranked"])
def test_matches_reference_ids(eg2, golden, tmp_path, name):
    tok = make_tokenizer(eg2, golden, name, str(tmp_path / f"{name}.gguf"))
    texts = unblob(golden["text"], golden["text_offsets"])
    ids, offs = golden[f"{name}_ids"], golden[f"{name}_id_offsets"]
    bad = []
    k = 0
    for t in texts:
        for add_special, parse_special in COMBOS:
            want = ids[offs[k]:offs[k + 1]]
            got = tok.encode(t, bool(add_special), bool(parse_special))
            if not np.array_equal(got, want):
                bad.append((t[:40], add_special, parse_special, want[:12].tolist(), got[:12].tolist()))
            k += 1
    tok.close()
    assert not bad, bad[:3]
    assert k == len(texts) * len(COMBOS) and len(texts) > 250


@pytest.mark.parametrize("threads", [1, 4])
def test_batch_packs_each_text(eg2, golden, tmp_path, threads):
    tok = make_tokenizer(eg2, golden, "spm", str(tmp_path / "spm.gguf"))
    texts = unblob(golden["text"], golden["text_offsets"])
    ids, offs = tok.encode_batch(texts, True, False, threads)
    assert offs[0] == 0 and offs[-1] == len(ids)
    for i, t in enumerate(texts):
        assert np.array_equal(ids[offs[i]:offs[i + 1]], tok.encode(t, True, False))
    tok.close()


def test_text_to_id_and_repeated_pieces(eg2, golden, tmp_path):
    tok = make_tokenizer(eg2, golden, "spm", str(tmp_path / "spm.gguf"))
    pieces = unblob(golden["spm_tokens"], golden["spm_token_offsets"])
    last = {}
    for i, p in enumerate(pieces):
        last[p if p else f"[EMPTY_{i}]".encode()] = i
    for p, i in list(last.items())[::37]:
        assert tok.text_to_id(p) == i
    assert tok.text_to_id(b"no such piece \x00") == -1
    tok.close()


def test_missing_byte_fallback_is_an_error(eg2, tmp_path):
    path = str(tmp_path / "bad.gguf")
    gguf_py.write_kv(path, [("tokenizer.ggml.tokens", "arr_str", [b"<pad>", b"<eos>", b"<bos>", b"<unk>", b"a"]),
                            ("tokenizer.ggml.scores", "arr_f32", np.zeros(5, np.float32)),
                            ("tokenizer.ggml.token_type", "arr_i32", np.array([3, 3, 3, 2, 1], np.int32))])
    with pytest.raises(eg2.HipError, match="byte fallback"):
        eg2.Tokenizer(path)
    gguf_py.write_kv(path, [("tokenizer.ggml.tokens", "arr_str", [b"a"])])
    with pytest.raises(eg2.HipError, match="missing tokenizer key"):
        eg2.Tokenizer(path)


def test_live_against_compiled_reference(eg2, golden, tmp_path):
    """Fresh random texts through both tokenizers, where oracle/_ref is built."""
    import ctypes as C

    ref_so = os.path.join(ROOT, "oracle", "_ref", "libref.so")
    if not os.path.exists(ref_so):
        pytest.skip("oracle/_ref is not built (no reference tree)")
    r = C.CDLL(ref_so)
    r.ref_tokenizer_open.restype = C.c_void_p
    r.ref_tokenizer_open.argtypes = [C.c_char_p]
    r.ref_tokenize.restype = C.c_size_t
    r.ref_tokenize.argtypes = [C.c_void_p, C.c_char_p, C.c_size_t, C.c_int, C.c_int, C.POINTER(C.c_int32),
                               C.c_size_t]
    r.ref_tokenizer_close.argtypes = [C.c_void_p]
    rng = np.random.default_rng(99)
    alphabet = list("abcdeABCDE \n\t.") + ["é", "中", "😀", "<bos>", "<start_of_turn>", "▁", "\xff"]
    buf = (C.c_int32 * 65536)()
    for name in ("spm", "ranked"):
        path = str(tmp_path / f"{name}.gguf")
        tok = make_tokenizer(eg2, golden, name, path)
        h = r.ref_tokenizer_open(path.encode())
        for _ in range(300):
            t = "".join(rng.choice(alphabet, size=rng.integers(0, 60))).encode("utf-8", "surrogateescape")
            for add_special, parse_special in COMBOS:
                n = r.ref_tokenize(h, t, len(t), add_special, parse_special, buf, 65536)
                assert np.array_equal(tok.encode(t, bool(add_special), bool(parse_special)), np.array(buf[:n])), t
        r.ref_tokenizer_close(h)
        tok.close()
