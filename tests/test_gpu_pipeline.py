"""The path end to end on the GPU at the benchmark workloads, against the
CPU oracle:

- the dynamic-batching stream of the benchmark (seed 42: requests of
  U{1..16} texts, lengths log-uniform in [4, 2048], dimensions cycling
  128/256/512/768) through eg2_stream_embed on the 24-layer model, its
  first requests up to a bounded token count;
- the 16x128 wave on the 24-layer model over several id seeds, reporting
  the parity margins;
- texts tokenized by eg2_tokenize_batch (bit-exact against the reference
  tokenizer's fixture ids) and packed straight into ei_gemma2_kfd_batch.

Bar (every embedding): cosine >= 0.9999 and max-abs <= 2e-3 against the
oracle, after the Matryoshka truncation and prefix L2 where the stream
applies it (kernels.c:393-407) -- and, since every kernel reproduces the
reference's arithmetic, bit-equality with the oracle."""
import json
import os
import sys

import numpy as np
import pytest

import gguf_py
import oracle_lib as OL

pytestmark = pytest.mark.gpu
COS_MIN, MAX_ABS = 0.9999, 2e-3
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
STREAM_TOKEN_BUDGET = 8192  # the oracle takes about a minute on 16 host threads


def oracle_waves(model, ids, offsets, threads=16):
    """Oracle embeddings of the texts [offsets[i], offsets[i+1]), packed
    greedily into oracle calls of at most 2048 tokens (a text's oracle
    result does not depend on its neighbours)."""
    n = len(offsets) - 1
    out = np.zeros((n, OL.N_EMBD), np.float32)
    i = 0
    while i < n:
        j = i + 1
        while j < n and offsets[j + 1] - offsets[i] <= OL.N_CTX:
            j += 1
        sub = np.asarray(offsets[i:j + 1], np.int64) - int(offsets[i])
        out[i:j] = OL.forward(model, ids[int(offsets[i]):int(offsets[j])], sub.astype(np.uint64), threads=threads)
        i = j
    return out


def margins(got, want):
    cos = (got * want).sum(1) / np.linalg.norm(got, axis=1) / np.linalg.norm(want, axis=1)
    return float(cos.min()), float(np.abs(got - want).max())


def test_config5_stream_against_oracle(eg2, gpu, full_model):
    sys.path.insert(0, ROOT)
    import bench

    ids, offsets, dims, texts = bench.config5_stream(eg2.VOCAB, with_requests=True)
    # The first requests whose texts fit the token budget.
    ends = np.cumsum(texts)
    r = int(np.searchsorted(offsets[ends], STREAM_TOKEN_BUDGET, side="right"))
    n_texts = int(ends[r - 1])
    offs = offsets[:n_texts + 1]
    sub_ids, sub_dims = ids[:int(offs[-1])], dims[:n_texts]
    enc = eg2.Encoder(full_model)
    try:
        out, waves = enc.stream(sub_ids, offs, sub_dims)
    finally:
        enc.close()
    want = oracle_waves(gguf_py.oracle_model(full_model), sub_ids, offs)
    worst_cos, worst_abs = 1.0, 0.0
    for i, d in enumerate(sub_dims):
        w = want[i].copy()
        assert OL.oracle().or_normalize_prefix(OL.fptr(w), int(d)) == 1
        c, a = margins(out[i:i + 1, :d], w[None, :d])
        worst_cos, worst_abs = min(worst_cos, c), max(worst_abs, a)
        assert not out[i, d:].any()
        assert np.array_equal(out[i, :d], w[:d]), i
    print(json.dumps({"config5_prefix": {"requests": r, "texts": n_texts, "tokens": int(offs[-1]), "waves": waves,
                                         "longest": int(np.diff(offs).max()), "min_cos": worst_cos,
                                         "max_abs": worst_abs}}))
    assert r >= 3 and waves >= 4
    assert worst_cos >= COS_MIN and worst_abs <= MAX_ABS


def stream_subset_against_oracle(eg2, enc, model, ids, offsets, dims, texts):
    """The stream on the given texts (indices into the config-5 text list),
    compared with the oracle after the Matryoshka prefix: (waves, min cos,
    max abs, bit-exact)."""
    lens = np.diff(offsets)[texts]
    sub_offs = np.concatenate([[0], np.cumsum(lens)])
    sub_ids = np.concatenate([ids[int(offsets[t]):int(offsets[t + 1])] for t in texts])
    sub_dims = dims[texts]
    out, waves = enc.stream(sub_ids, sub_offs, sub_dims)
    want = oracle_waves(model, sub_ids, sub_offs)
    cos, mx, exact = 1.0, 0.0, True
    for i, d in enumerate(sub_dims):
        w = want[i].copy()
        assert OL.oracle().or_normalize_prefix(OL.fptr(w), int(d)) == 1
        c, a = margins(out[i:i + 1, :d], w[None, :d])
        cos, mx = min(cos, c), max(mx, a)
        exact = exact and bool(np.array_equal(out[i, :d], w[:d])) and not out[i, d:].any()
    return waves, cos, mx, exact


def test_config5_long_request_and_full_wave_against_oracle(eg2, gpu, full_model):
    """Three more pieces of the config-5 stream against the oracle: the
    first request holding a text of at least 1,900 tokens (all of its
    texts); the most populous wave of the batcher's packing of the whole
    stream (25 sequences: its log-uniform lengths never fill 32); and 32
    texts of the stream that make a full 32-sequence wave (the first 32 of
    at most 64 tokens), each embedded as its own stream (the packer keeps
    each of the last two in one wave)."""
    sys.path.insert(0, ROOT)
    import bench

    ids, offsets, dims, texts = bench.config5_stream(eg2.VOCAB, with_requests=True)
    lens = np.diff(offsets)
    ends = np.cumsum(texts)
    starts = ends - texts
    long_req = next(r for r in range(len(texts)) if lens[starts[r]:ends[r]].max() >= 1900)
    req_texts = list(range(int(starts[long_req]), int(ends[long_req])))
    wave_texts = sorted(max(eg2.pack_waves(lens), key=len))
    full_texts = [int(t) for t in np.flatnonzero(lens <= 64)[:32]]
    model = gguf_py.oracle_model(full_model)
    enc = eg2.Encoder(full_model)
    rows = {}
    try:
        for name, sel in (("long_request", req_texts), ("largest_wave", wave_texts), ("full_wave", full_texts)):
            waves, c, a, exact = stream_subset_against_oracle(eg2, enc, model, ids, offsets, dims, sel)
            rows[name] = {"texts": len(sel), "tokens": int(lens[sel].sum()), "longest": int(lens[sel].max()),
                          "waves": waves, "min_cos": c, "max_abs": a, "bit_exact": exact}
    finally:
        enc.close()
    print(json.dumps({"config5_more": {"request": int(long_req), **rows}}))
    assert rows["long_request"]["longest"] >= 1900
    assert rows["largest_wave"]["texts"] >= 25 and rows["largest_wave"]["waves"] == 1
    assert rows["full_wave"]["texts"] == 32 and rows["full_wave"]["waves"] == 1
    for row in rows.values():
        assert row["min_cos"] >= COS_MIN and row["max_abs"] <= MAX_ABS and row["bit_exact"], row


def test_config4_margins_over_seeds(eg2, gpu, full_model):
    """The 16x128 wave with five more id seeds: every seed within the bar,
    margins printed for the record."""
    enc = eg2.Encoder(full_model)
    model = gguf_py.oracle_model(full_model)
    offsets = np.arange(0, 16 * 128 + 1, 128)
    rows = []
    try:
        for seed in range(1, 6):
            ids = np.random.default_rng(seed).integers(0, OL.VOCAB, 16 * 128).astype(np.int32)
            got = enc.batch(ids, offsets)
            want = OL.forward(model, ids, offsets.astype(np.uint64), threads=16)
            c, a = margins(got, want)
            rows.append({"seed": seed, "min_cos": c, "max_abs": a, "bit_exact": bool(np.array_equal(got, want))})
    finally:
        enc.close()
    print(json.dumps({"config4_seeds": rows}))
    for row in rows:
        assert row["min_cos"] >= COS_MIN and row["max_abs"] <= MAX_ABS and row["bit_exact"], row


def test_tokenized_texts_through_the_executor(eg2, gpu, tmp_path_factory):
    """eg2_tokenize_batch on the fixture texts gives the reference
    tokenizer's ids bit for bit (tokenizer.c:574-631, add_special on,
    parse_special off); the ids and their offsets go straight into
    ei_gemma2_kfd_batch as the service hands them over
    (inference_service.c:1156-1189), and the embeddings match the oracle."""
    from test_tokenizer_cpu import GOLDEN, make_tokenizer, unblob

    g = np.load(GOLDEN)
    d = tmp_path_factory.mktemp("tok")
    tok = make_tokenizer(eg2, g, "spm", str(d / "spm.gguf"))
    texts = unblob(g["text"], g["text_offsets"])
    want_ids, want_offs = g["spm_ids"], g["spm_id_offsets"]
    try:
        ids, offs = tok.encode_batch(texts, True, False, 8)
    finally:
        tok.close()
    # Fixture order: per text, the (add_special, parse_special) pairs
    # (1,0), (1,1), (0,0), (0,1); (1,0) is the first of each text's four.
    for i in range(len(texts)):
        k = 4 * i
        assert np.array_equal(ids[offs[i]:offs[i + 1]], want_ids[want_offs[k]:want_offs[k + 1]]), i
    # The longest prefix of texts that fits one 2048-token wave.
    n = int(np.searchsorted(offs, OL.N_CTX, side="right")) - 1
    assert n >= 20
    wave_offs = offs[:n + 1]
    path = str(d / "model.gguf")
    eg2.synth_gguf(path, seed=41, n_layer=2, dense_head=True, sliding_window=512, sliding_window_pattern=2,
                   rope_base_full=1e6, rope_base_swa=1e4, threads=16)
    enc = eg2.Encoder(path)
    try:
        got = enc.batch(ids[:wave_offs[-1]], wave_offs)
    finally:
        enc.close()
    want = OL.forward(gguf_py.oracle_model(path), ids[:wave_offs[-1]], wave_offs.astype(np.uint64), threads=16)
    c, a = margins(got, want)
    print(json.dumps({"tokenized_wave": {"texts": n, "tokens": int(wave_offs[-1]), "min_cos": c, "max_abs": a}}))
    assert c >= COS_MIN and a <= MAX_ABS
    assert np.array_equal(got, want)


def test_requests_against_the_http_parity_contract(eg2, gpu, tmp_path_factory):
    """The checks of the reference's tests/http_parity.py:15-107 on the
    request path without its HTTP transport, as the server's handle_embed
    runs it (server.c:1029-1210): the texts of a request tokenized by
    eg2_tokenize_batch, embedded 768 wide by eg2_stream_embed (the service
    hands the server full embeddings), and the OpenAI response body written
    by eg2_embeddings_response (prefix L2 to `dimensions`, float text or
    base64), then parsed as JSON. Where http_parity.py compares the GPU
    server with the CPU server by cosine >= 0.99, the body here is compared
    byte for byte with the body written from the oracle's embeddings;
    batch = solo, reversed order and concurrent requests are asserted bit
    for bit (the script: cosine >= 0.99999)."""
    import base64
    import math
    import struct
    import threading

    from test_tokenizer_cpu import GOLDEN, make_tokenizer

    g = np.load(GOLDEN)
    d = tmp_path_factory.mktemp("req")
    tok = make_tokenizer(eg2, g, "spm", str(d / "spm.gguf"))
    path = str(d / "model.gguf")
    eg2.synth_gguf(path, seed=43, n_layer=2, dense_head=True, sliding_window=512, sliding_window_pattern=2,
                   rope_base_full=1e6, rope_base_swa=1e4, threads=16)
    model = gguf_py.oracle_model(path)
    enc = eg2.Encoder(path)
    lock = threading.Lock()  # the tokenizer handle is used from one thread at a time

    def embed(texts, dims=768, encoding="float", oracle=False):
        """One request: (response body, prompt tokens); raises on a rejected request."""
        raw = [t.encode() for t in ([texts] if isinstance(texts, str) else texts)]
        with lock:
            ids, offs = tok.encode_batch(raw, True, False, 4)
        if oracle:
            e = oracle_waves(model, ids, offs)
        else:
            e, _ = enc.stream(ids, offs, [768] * len(raw))
        body = eg2.embeddings_response(e, dims, api="openai", encoding=encoding, model="embeddinggemma-2",
                                       prompt_tokens=int(offs[-1]))
        return body, int(offs[-1])

    def request(texts, dims=768, encoding="float"):
        """http_parity.py:15-34 on the parsed body."""
        body, tokens = embed(texts, dims, encoding)
        obj = json.loads(body)
        assert obj["object"] == "list"
        assert obj["usage"]["total_tokens"] == obj["usage"]["prompt_tokens"] == tokens > 0
        vectors = []
        for i, item in enumerate(obj["data"]):
            assert item["index"] == i and item["object"] == "embedding"
            v = item["embedding"]
            if encoding == "base64":
                v = struct.unpack("<" + "f" * dims, base64.b64decode(v, validate=True))
            assert len(v) == dims and all(math.isfinite(x) for x in v)
            assert abs(math.sqrt(sum(x * x for x in v)) - 1) < 1e-4
            vectors.append(np.array(v, np.float32))
        assert len(vectors) == (1 if isinstance(texts, str) else len(texts))
        return np.stack(vectors), body

    try:
        texts = ["", "hello world", "检索增强生成与向量数据库。", "a " * 37,
                 "query: How does a GPU execute a kernel?", "emoji: 🌍 café\nsecond line"]
        # http_parity.py --long: a sequence past 1024 tokens, within one wave
        reps = 1030
        while len(tok.encode(("boundary " * reps).encode(), True, False)) > 2000:
            reps -= 40
        long_texts = ["boundary " * reps, "short unrelated sequence"]
        assert len(tok.encode(long_texts[0].encode(), True, False)) > 1024
        wide = [f"wide item {j}: " + "word " * (27 + j % 7) for j in range(16)]
        for group in (texts, long_texts, wide):
            got, body = request(group)
            assert body == embed(group, oracle=True)[0]  # the CPU side, byte for byte
            for text, vector in zip(group, got):
                assert np.array_equal(request(text)[0][0], vector)
            rev, _ = request(list(reversed(group)))
            assert np.array_equal(rev[::-1], got)
        for dim in (128, 256, 512, 768):
            f, _ = request("format test", dim)
            b, _ = request("format test", dim, "base64")
            assert np.array_equal(f, b)
        full, _ = request(texts)
        results, errors = [None] * len(texts), []

        def one(i):
            try:
                results[i] = request(texts[i])[0][0]
            except Exception as e:  # reported below
                errors.append(repr(e))

        threads = [threading.Thread(target=one, args=(i,)) for i in range(len(texts))]
        for t in threads:
            t.start()
        for t in threads:
            t.join(timeout=90)
        assert not errors and all(r is not None for r in results), errors
        assert all(np.array_equal(r, v) for r, v in zip(results, full))
        # invalid requests: no input, unsupported dimensions, a text over 2048 tokens
        with pytest.raises(eg2.HipError, match="invalid"):
            embed([])
        with pytest.raises(ValueError, match="dims"):
            embed("test", 17)
        with pytest.raises(eg2.HipError, match="1..2048"):
            embed("word " * 2100)
        request("still healthy after validation failures")
    finally:
        enc.close()
        tok.close()
