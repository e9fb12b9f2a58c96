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
