"""The dynamic-batching stream (eg2_stream_embed) on the GPU: texts packed
into waves by the batcher's rules, each wave through the executor, each
embedding truncated and prefix-normalised (kernels.c:393-407)."""
import numpy as np
import pytest

import gguf_py
import oracle_lib as OL

pytestmark = pytest.mark.gpu
DIMS = [128, 256, 512, 768]


@pytest.fixture(scope="module")
def stream_encoder(eg2, gpu, tmp_path_factory):
    path = str(tmp_path_factory.mktemp("s") / "stream.gguf")
    eg2.synth_gguf(path, seed=31, n_layer=2, dense_head=True, sliding_window=512, sliding_window_pattern=2,
                   rope_base_full=1e6, rope_base_swa=1e4, threads=16)
    enc = eg2.Encoder(path)
    yield enc, path
    enc.close()


def make_stream(rng, n_texts, max_len):
    lens = np.floor(np.exp(rng.uniform(np.log(1), np.log(max_len), n_texts))).astype(int)
    offsets = np.concatenate([[0], np.cumsum(lens)])
    ids = rng.integers(0, OL.VOCAB, int(offsets[-1])).astype(np.int32)
    dims = [DIMS[i % 4] for i in range(n_texts)]
    return ids, offsets, dims


def test_stream_equals_each_text_alone(eg2, stream_encoder):
    """Packing never changes a sequence's bits, so every stream embedding
    equals the text run alone, truncated and prefix-normalised."""
    enc, _ = stream_encoder
    rng = np.random.default_rng(7)
    ids, offsets, dims = make_stream(rng, 70, 700)
    cfg = eg2.batch_config(max_batch_requests=8)
    out, waves = enc.stream(ids, offsets, dims, cfg)
    lengths = np.diff(offsets).tolist()
    assert waves == len(eg2.pack_waves(lengths, cfg)) > 1
    for i in range(len(dims)):
        alone = enc.batch(ids[offsets[i]:offsets[i + 1]], [0, lengths[i]])[0]
        want = eg2.normalize_prefix(alone, dims[i])
        assert np.array_equal(out[i, :dims[i]], want[:dims[i]]), i
        assert not out[i, dims[i]:].any()
        assert abs(np.linalg.norm(out[i, :dims[i]]) - 1) < 1e-5


def test_stream_matches_oracle(eg2, stream_encoder):
    """A small stream against the CPU oracle: every truncated, normalised
    embedding within cosine >= 0.9999 and max-abs <= 2e-3, and equal bit for
    bit."""
    enc, path = stream_encoder
    rng = np.random.default_rng(8)
    ids, offsets, dims = make_stream(rng, 12, 120)
    out, _ = enc.stream(ids, offsets, dims)
    want = OL.forward(gguf_py.oracle_model(path), ids, offsets.astype(np.uint64), threads=16)
    for i, d in enumerate(dims):
        w = want[i].copy()
        assert OL.oracle().or_normalize_prefix(OL.fptr(w), d) == 1
        g = out[i, :d]
        cos = float(g @ w[:d] / np.linalg.norm(g) / np.linalg.norm(w[:d]))
        assert cos >= 0.9999 and np.abs(g - w[:d]).max() <= 2e-3, (i, cos)
        assert np.array_equal(g, w[:d]), i


def test_stream_rejects_bad_texts(eg2, stream_encoder):
    enc, _ = stream_encoder
    with pytest.raises(eg2.HipError, match="dimensions"):
        enc.stream(np.zeros(4, np.int32), [0, 4], [100])
    with pytest.raises(eg2.HipError, match="empty"):
        enc.stream(np.zeros(4, np.int32), [0, 4, 4], [128, 128])
    with pytest.raises(eg2.HipError, match="out of range"):
        enc.stream(np.full(4, OL.VOCAB, np.int32), [0, 4], [128])
    # the context is poisoned only by device failures, not by rejected input
    out, _ = enc.stream(np.zeros(4, np.int32), [0, 4], [768])
    assert abs(np.linalg.norm(out[0]) - 1) < 1e-5


def test_concurrent_streams_and_batches(eg2, stream_encoder):
    """Streams of many waves and batch calls from several threads at once on
    one context: each stream takes one lane waiting and the others only if
    free, so no thread waits while holding lanes another one waits for;
    every result equals the one-at-a-time result."""
    import threading

    enc, _ = stream_encoder
    rng = np.random.default_rng(9)
    streams = [make_stream(rng, 40, 600) for _ in range(3)]
    cfg = eg2.batch_config(max_batch_requests=4)
    alone = [enc.stream(ids, offs, dims, cfg)[0] for ids, offs, dims in streams]
    ids_b, offs_b, _ = streams[0]
    batch_alone = enc.batch(ids_b[:offs_b[5]], offs_b[:6])
    errors = []

    def run_stream(k):
        try:
            for _ in range(2):
                got, waves = enc.stream(*streams[k], cfg)
                if waves < enc.lanes or not np.array_equal(got, alone[k]):
                    errors.append(("stream", k, waves))
        except Exception as e:  # reported below
            errors.append(repr(e))

    def run_batches():
        try:
            for _ in range(6):
                if not np.array_equal(enc.batch(ids_b[:offs_b[5]], offs_b[:6]), batch_alone):
                    errors.append("batch")
        except Exception as e:  # reported below
            errors.append(repr(e))

    threads = [threading.Thread(target=run_stream, args=(k,)) for k in range(3)]
    threads += [threading.Thread(target=run_batches) for _ in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=90)
    assert not any(t.is_alive() for t in threads), "a thread did not finish"
    assert not errors, errors
