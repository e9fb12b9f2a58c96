"""Writes tests/golden/reference_vectors.npz: seeded inputs and the outputs of
the reference's own CPU functions (vendor/embeddinggemma.c/src/quants.c,
kernels.c and the Q8_0 x Q8_0 `mm` of gemma2.c), compiled from the reference
tree by oracle/Makefile into oracle/_ref/libref.so; and
tests/golden/float_text.npz, float32 values and their text by the
reference's float_format.c.

Run where the reference tree is present:
    make -C oracle ref && python tests/golden/make_golden.py
The fixture holds data only (inputs and expected outputs).
"""
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(HERE)), "oracle"))
from oracle_lib import Q8, fptr, ref, vptr  # noqa: E402


def main():
    r = ref()
    if r is None:
        raise SystemExit("oracle/_ref/libref.so is not built (make -C oracle ref)")
    rng = np.random.default_rng(20260101)
    out = {}

    # fp16 conversion (quants.c:13-37): specials, ties, subnormals, random.
    special = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.0, 65520.0, 65536.0, 70000.0, 1e-8, 2.98e-8,
                        2.9802322e-8, 5.96e-8, 6.1e-5, 6.097555e-5, np.inf, -np.inf, np.nan, 0.5 + 2 ** -12,
                        1.0 + 2 ** -11, 1.0 + 3 * 2 ** -12, 2049.0, 2051.0], dtype=np.float32)
    rand = (rng.standard_normal(4000) * 10.0 ** rng.integers(-8, 5, 4000)).astype(np.float32)
    f16_in = np.concatenate([special, rand])
    out["fp16_in"] = f16_in
    out["fp16_out"] = np.array([r.ei_fp32_to_fp16(float(v)) for v in f16_in], dtype=np.uint16)

    # Q8_0 quantizer (quants.c:97-177): random scales plus edge rows.
    x = (rng.standard_normal((48, 64)) * 10.0 ** rng.uniform(-4, 3, (48, 1))).astype(np.float32)
    x[0] = 0.0
    x[1, :32] = 0.5
    x[1, 32:] = np.float32(127.0 / 2)
    x[2] = np.arange(64, dtype=np.float32) - 31.5
    x[3, :] = 1e-30
    qb = np.zeros((48, 2), dtype=Q8)
    for i in range(48):
        r.ei_quantize_row_q8_0(fptr(x[i]), vptr(qb[i]), 64)
    out["quant_in"], out["quant_out"] = x, qb.view(np.uint8).reshape(48, 68)

    # RMSNorm variants on 768-wide rows (kernels.c:139-188).
    rows = (rng.standard_normal((6, 768)) * rng.uniform(0.1, 30, (6, 1))).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(768)).astype(np.float32)
    h = (rng.standard_normal((6, 768)) * 2).astype(np.float32)
    norm = np.zeros_like(rows)
    nq = np.zeros((6, 24), dtype=Q8)
    resid = rows.copy()
    for i in range(6):
        r.ei_rms_norm(fptr(rows[i]), fptr(w), 768, 1e-6, fptr(norm[i]))
        r.ei_rms_norm_quantize_q8_0(fptr(rows[i]), fptr(w), 768, 1e-6, vptr(nq[i]))
        r.ei_rms_norm_residual_inplace(fptr(resid[i]), fptr(h[i]), fptr(w), 768, 1e-6)
    out.update(norm_x=rows, norm_w=w, norm_h=h, norm_out=norm, norm_q8=nq.view(np.uint8).reshape(6, 816),
               resid_out=resid)

    # QK-norm + RoPE + q scale (kernels.c:233-264).
    qw = (1.0 + 0.1 * rng.standard_normal(256)).astype(np.float32)
    kw = (1.0 + 0.1 * rng.standard_normal(256)).astype(np.float32)
    cases = [(0, 10000.0), (1, 10000.0), (127, 10000.0), (2047, 10000.0), (511, 1000000.0), (1500, 1000000.0)]
    q_in = rng.standard_normal((len(cases), 768)).astype(np.float32)
    k_in = rng.standard_normal((len(cases), 256)).astype(np.float32)
    q_out, k_out = q_in.copy(), k_in.copy()
    for i, (p, base) in enumerate(cases):
        r.ei_qk_norm_rope_qk_inplace(fptr(q_out[i]), fptr(k_out[i]), fptr(qw), fptr(kw), p, base, 1e-6)
    out.update(qk_qw=qw, qk_kw=kw, qk_pos=np.array([c[0] for c in cases], np.int32),
               qk_base=np.array([c[1] for c in cases], np.float32), qk_q_in=q_in, qk_k_in=k_in, qk_q_out=q_out,
               qk_k_out=k_out)

    # Attention over one sequence, full and windowed (kernels.c:324-360).
    T = 24
    aq = (rng.standard_normal((T, 768)) * 0.3).astype(np.float32)
    ak = rng.standard_normal((T, 256)).astype(np.float32)
    av = rng.standard_normal((T, 256)).astype(np.float32)
    scores = np.zeros(4096, np.float32)
    att = {}
    for win in (0, 8):
        ctx = np.zeros((T, 768), np.float32)
        r.ei_attention_mha_range(fptr(aq), fptr(ak), fptr(av), T, win, 0, T, fptr(ctx), fptr(scores))
        att[win] = ctx
    out.update(att_q=aq, att_k=ak, att_v=av, att_full=att[0], att_win8=att[8])

    # GELU (kernels.c:367-371) and GeGLU + Q8_0 (kernels.c:377-391).
    gx = (rng.standard_normal(2000) * 4).astype(np.float32)
    out["gelu_in"] = gx
    out["gelu_out"] = np.array([r.ei_gelu_tanh(float(v)) for v in gx], np.float32)
    gate = (rng.standard_normal((3, 1152)) * 2).astype(np.float32)
    up = rng.standard_normal((3, 1152)).astype(np.float32)
    gq = np.zeros((3, 36), dtype=Q8)
    for i in range(3):
        r.ei_gelu_mul_quantize_q8_0(fptr(gate[i]), fptr(up[i]), 1152, vptr(gq[i]))
    out.update(geglu_gate=gate, geglu_up=up, geglu_q8=gq.view(np.uint8).reshape(3, 36 * 34))

    # L2 and Matryoshka prefixes (kernels.c:393-407), mean pool (:417-427).
    e = rng.standard_normal((4, 768)).astype(np.float32)
    pref = np.zeros((4, 4, 768), np.float32)
    for i in range(4):
        for j, dims in enumerate((128, 256, 512, 768)):
            v = e[i].copy()
            assert r.ei_embedding_normalize_prefix(fptr(v), dims)
            pref[i, j] = v
    l2 = e.copy()
    for i in range(4):
        r.ei_l2_normalize(fptr(l2[i]), 768)
    px = (rng.standard_normal((5, 768)) * 3).astype(np.float32)
    pooled = np.zeros(768, np.float32)
    r.ei_mean_pool_rms_l2(fptr(px.copy()), 5, fptr(w), 1e-6, fptr(pooled))
    out.update(l2_in=e, l2_out=l2, prefix_out=pref, pool_x=px, pool_out=pooled)

    # Q8_0 x Q8_0 projection (gemma2.c:142-153: quantize x, block dots).
    for name, (n, k, m) in {"mm_a": (5, 64, 7), "mm_b": (4, 768, 16)}.items():
        wf = (rng.standard_normal((m, k)) * 0.02).astype(np.float32)
        wq = np.zeros((m, k // 32), dtype=Q8)
        for i in range(m):
            r.ei_quantize_row_q8_0(fptr(wf[i]), vptr(wq[i]), k)
        xf = rng.standard_normal((n, k)).astype(np.float32)
        y = np.zeros((n, m), np.float32)
        r.ref_mm_q8_0(vptr(wq), k, m, fptr(xf), n, fptr(y))
        out[name + "_w"] = wq.view(np.uint8).reshape(m, k // 32 * 34)
        out[name + "_x"], out[name + "_y"] = xf, y

    # Embedding rows (engine.c:288-295).
    tab = np.zeros((4, 24), dtype=Q8)
    tf = (rng.standard_normal((4, 768)) * 0.05).astype(np.float32)
    for i in range(4):
        r.ei_quantize_row_q8_0(fptr(tf[i]), vptr(tab[i]), 768)
    emb = np.zeros((4, 768), np.float32)
    for i in range(4):
        r.ref_embed_row(vptr(tab), 4, i, fptr(emb[i]))
    out.update(embed_table=tab.view(np.uint8).reshape(4, 816), embed_out=emb)

    path = os.path.join(HERE, "reference_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")
    float_text(r, rng)
    tokenizer_vectors(r)


SP = "\u2581"
ALPHABET = list("abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOP0123456789.,;:!?'-()") + ["é", "ü", "中", "文", "😀",
                                                                                   "\t", "\n", SP]
COMBOS = [(1, 0), (1, 1), (0, 0), (0, 1)]  # (add_special, parse_special)


def synth_vocab(rng, ranked, words):
    """A seeded SentencePiece-style vocabulary exercising every branch of the
    reference tokenizer: control / unknown / user-defined specials (one a
    prefix of another, one empty piece), byte pieces (some bytes only as raw
    one-byte pieces), single characters (some missing, so they fall back to
    bytes), corpus substrings with many equal scores, repeated pieces, and
    in the ranked mode newline pieces and merge rules (repeated ones, and
    rules whose joined text is not a piece)."""
    tokens = [b"<pad>", b"<eos>", b"<bos>", b"<unk>", b"<start_of_turn>", b"<end_of_turn>", b"<mask>", b"<start",
              b""]
    types = [3, 3, 3, 2, 4, 4, 3, 4, 1]
    raw_bytes = set(b"abcdefgh")
    for b in range(256):
        if b not in raw_bytes:
            tokens.append(f"<0x{b:02X}>".encode())
            types.append(6)
    missing = {"Q", "z", "😀", "文"}
    singles = [c for c in ALPHABET if c not in missing]
    tokens += [c.encode() for c in singles]
    types += [1] * len(singles)
    subs = set()
    for w in words:
        t = SP + w
        for i in range(len(t)):
            for j in range(i + 2, min(len(t), i + 6) + 1):
                if rng.random() < 0.5:
                    subs.add(t[i:j])
    subs = sorted(subs)
    tokens += [x.encode() for x in subs]
    types += [1] * len(subs)
    if ranked:
        tokens += [b"\n", b"\n\n", b"\n\n\n"]
        types += [1, 1, 1]
    for i in rng.integers(300, len(tokens), 20):  # repeated pieces: the last id wins
        tokens.append(tokens[int(i)])
        types.append(types[int(i)])
    scores = (-rng.integers(0, 40, len(tokens)) / 4.0).astype(np.float32)
    scores[:9] = 0.0
    merges = []
    if ranked:
        pieces = set(subs) | set(singles)
        for x in subs:
            cut = int(rng.integers(1, len(x)))
            if x[:cut] in pieces and x[cut:] in pieces:
                merges.append(f"{x[:cut]} {x[cut:]}".encode())
        for _ in range(200):  # rules whose joined text is not a piece
            a, b = rng.choice(singles[:40], 2)
            merges.append(f"{a} {b}".encode())
        rng.shuffle(merges)
        merges += merges[:30]  # repeated rules: the first rank wins
    return tokens, types, scores, merges


def synth_texts(rng, vocab_words):
    fixed = [b"", b" ", b"a", b"hello world", b"  two  spaces ", b"<bos>x<eos>",
             b"pre<start_of_turn>mid<end_of_turn>post", b"<start_of", b"<start<start_of_turn>", b"<unk>", b"<mask>",
             "\u03a9mega \x01 ctrl".encode(), b"\xff\xfe bad utf8 \xc3", "中文 😀 émoji".encode(),
             b"tab\tand\nnewline\n\n\n x", b"\n\n", "\u2581literal".encode(), b"QzQz zz", b"aaaaaaaaaaaaaaaa",
             b"abcdefgh hgfedcba"]
    words = [w for w in "the quick brown fox jumps over lazy dog cafe naive 中文 😀 émoji abc ab ba".split()]
    chars = ALPHABET + ["Ω", "\x01", " "]
    out = list(fixed)
    for i in range(260):
        parts = []
        for _ in range(int(rng.integers(1, 25))):
            u = rng.random()
            if u < 0.6:
                parts.append(str(rng.choice(words)))
            elif u < 0.85:
                parts.append("".join(rng.choice(chars, size=rng.integers(1, 6))))
            elif u < 0.95:
                parts.append(str(rng.choice(["<bos>", "<eos>", "<unk>", "<mask>", "<start_of_turn>", "<start"])))
            else:
                parts.append("\n" * int(rng.integers(1, 4)))
        sep = [" ", "  ", "", "\t"]
        out.append("".join(p + str(rng.choice(sep, p=[0.7, 0.1, 0.15, 0.05])) for p in parts).encode())
    for i in range(120):  # texts of the vocabularies' own words: long merges
        out.append(" ".join(str(w) for w in rng.choice(vocab_words, size=rng.integers(1, 30))).encode())
    out.append(" ".join(str(rng.choice(words)) for _ in range(900)).encode())  # a long text
    return out


def blob(items):
    offs = np.concatenate([[0], np.cumsum([len(x) for x in items])]).astype(np.int64)
    return np.frombuffer(b"".join(items), np.uint8) if offs[-1] else np.zeros(0, np.uint8), offs


def tokenizer_vectors(r):
    """tests/golden/tokenizer_vectors.npz: three synthetic vocabularies (the
    vocabulary and model flags as data), seeded texts, and the ids the
    reference's tokenizer.c gives each text under each (add_special,
    parse_special) pair."""
    import tempfile

    import gguf_py

    r.ref_tokenizer_open.restype = C.c_void_p
    r.ref_tokenizer_open.argtypes = [C.c_char_p]
    r.ref_tokenize.restype = C.c_size_t
    r.ref_tokenize.argtypes = [C.c_void_p, C.c_char_p, C.c_size_t, C.c_int, C.c_int, C.POINTER(C.c_int32),
                               C.c_size_t]
    r.ref_tokenizer_close.argtypes = [C.c_void_p]
    rng = np.random.default_rng(20260201)
    letters = list("abcdefghijklmnopqrstuvwxyzABCDE") + ["é", "ü", "中"]
    words = ["".join(rng.choice(letters, size=rng.integers(1, 8))) for _ in range(300)]
    texts = synth_texts(rng, words)
    out = {}
    out["text"], out["text_offsets"] = blob(texts)
    configs = {"spm": dict(ranked=False, bos=2, eos=1, add_bos=True, add_eos=False, prefix=True),
               "spm_eos": dict(ranked=False, bos=4, eos=6, add_bos=False, add_eos=True, prefix=False),
               "ranked": dict(ranked=True, bos=2, eos=1, add_bos=True, add_eos=True, prefix=True)}
    for name, c in configs.items():
        tokens, types, scores, merges = synth_vocab(rng, c["ranked"], words)
        kvs = [("tokenizer.ggml.model", "str", "llama"), ("tokenizer.ggml.tokens", "arr_str", tokens),
               ("tokenizer.ggml.scores", "arr_f32", scores), ("tokenizer.ggml.token_type", "arr_i32", types),
               ("tokenizer.ggml.bos_token_id", "u32", c["bos"]), ("tokenizer.ggml.eos_token_id", "u32", c["eos"]),
               ("tokenizer.ggml.add_bos_token", "bool", c["add_bos"]),
               ("tokenizer.ggml.add_eos_token", "bool", c["add_eos"]),
               ("tokenizer.ggml.add_space_prefix", "bool", c["prefix"])]
        if merges:
            kvs.append(("tokenizer.ggml.merges", "arr_str", merges))
        with tempfile.TemporaryDirectory() as d:
            path = os.path.join(d, "tok.gguf")
            gguf_py.write_kv(path, kvs)
            h = r.ref_tokenizer_open(path.encode())
            ids, offs = [], [0]
            buf = (C.c_int32 * 65536)()
            for t in texts:
                for add_special, parse_special in COMBOS:
                    n = r.ref_tokenize(h, t, len(t), add_special, parse_special, buf, 65536)
                    assert n <= 65536
                    ids.extend(buf[:n])
                    offs.append(offs[-1] + n)
            r.ref_tokenizer_close(h)
        out[f"{name}_tokens"], out[f"{name}_token_offsets"] = blob(tokens)
        out[f"{name}_types"] = np.array(types, np.int32)
        out[f"{name}_scores"] = scores
        out[f"{name}_merges"], out[f"{name}_merge_offsets"] = blob(merges)
        out[f"{name}_flags"] = np.array([c["bos"], c["eos"], c["add_bos"], c["add_eos"], c["prefix"]], np.int32)
        out[f"{name}_ids"] = np.array(ids, np.int32)
        out[f"{name}_id_offsets"] = np.array(offs, np.int64)
    path = os.path.join(HERE, "tokenizer_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(texts)} texts x {len(COMBOS)} flag pairs x "
          f"{len(configs)} vocabularies)")


def float_text(r, rng):
    """tests/golden/float_text.npz: float32 bit patterns and their text by the
    reference's ei_f32_to_chars (float_format.c:276-308): specials, binade
    bottoms and tops, subnormals, powers of ten, random bit patterns and
    embedding-like values; strings as one byte blob with offsets."""
    r.ei_f32_to_chars.restype = C.c_size_t
    r.ei_f32_to_chars.argtypes = [C.c_char_p, C.c_float]
    special = [0x00000000, 0x80000000, 0x00000001, 0x80000001, 0x007FFFFF, 0x00800000, 0x00800001, 0x7F7FFFFF,
               0xFF7FFFFF, 0x3F800000, 0x3F7FFFFF, 0x3F800001, 0x4B000000, 0x4B7FFFFF, 0x3DCCCCCD, 0x3E800000]
    edges = []
    for ef in range(1, 255, 3):  # binade bottoms and their neighbours
        base = ef << 23
        edges += [base, base + 1, base - 1 if ef > 1 else base + 2, base | 0x7FFFFF]
    tens = np.float32(10.0) ** np.arange(-45, 39, dtype=np.float64)
    tens = tens[np.isfinite(tens)].astype(np.float32).view(np.uint32).tolist()
    halves = (np.arange(1, 2000, dtype=np.float32) * np.float32(0.5)).view(np.uint32).tolist()
    rand_bits = rng.integers(0, 2 ** 32, 12000, dtype=np.uint64).astype(np.uint32).tolist()
    emb = (rng.standard_normal(12000) / np.sqrt(768)).astype(np.float32).view(np.uint32).tolist()
    bits = np.array(special + edges + tens + halves + rand_bits + emb, dtype=np.uint32)
    bits = bits[np.isfinite(bits.view(np.float32))]
    buf = C.create_string_buffer(64)
    texts, offs = [], [0]
    for b in bits:
        n = r.ei_f32_to_chars(buf, float(np.uint32(b).view(np.float32)))
        texts.append(buf.raw[:n])
        offs.append(offs[-1] + n)
    path = os.path.join(HERE, "float_text.npz")
    np.savez_compressed(path, bits=bits, text=np.frombuffer(b"".join(texts), np.uint8),
                        offsets=np.array(offs, np.int64))
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(bits)} values)")


if __name__ == "__main__":
    main()
