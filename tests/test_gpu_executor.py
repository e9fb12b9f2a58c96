"""End-to-end parity of the executor ABI (ei_gemma2_kfd_create/_batch/_free)
against the CPU oracle, on synthetic Q8_0 gemma-embedding models.

Bar: per-embedding cosine >= 0.9999 and max-abs <= 2e-3
against the oracle on the same seeded weights and ids (fp32 embeddings); every
kernel reproduces the reference's arithmetic, so the embeddings are in fact
asserted equal to the oracle's bit for bit."""
import os
import time

import numpy as np
import pytest

import gguf_py
import oracle_lib as OL

pytestmark = pytest.mark.gpu
COS_MIN, MAX_ABS = 0.9999, 2e-3


def cosines(a, b):
    return (a * b).sum(1) / np.linalg.norm(a, axis=1) / np.linalg.norm(b, axis=1)


@pytest.fixture(scope="module")
def small_model(eg2, tmp_path_factory):
    path = str(tmp_path_factory.mktemp("m") / "small.gguf")
    # Real-model attention pattern: SWA (window 512, base 1e4) except every
    # 3rd layer full (base 1e6), plus the dense head.
    eg2.synth_gguf(path, seed=21, n_layer=3, dense_head=True, sliding_window=512, sliding_window_pattern=3,
                   rope_base_full=1e6, rope_base_swa=1e4, threads=16)
    return path


@pytest.fixture(scope="module")
def small_encoder(eg2, gpu, small_model):
    enc = eg2.Encoder(small_model)
    yield enc
    enc.close()


def run_oracle(path, ids, offsets):
    return OL.forward(gguf_py.oracle_model(path), ids, np.asarray(offsets, np.uint64), threads=16)


@pytest.mark.parametrize("lens", [[5], [1, 1, 1], [37, 3, 100, 1, 64], [200, 50, 9], [400, 7, 90], [700, 300, 1],
                                  [2048]])
def test_small_model_parity(small_encoder, small_model, lens):
    """3-layer model, several packings (single token, many tiny sequences,
    ragged, long, one full 2048-token wave; their longest sequences pick
    each of the softmax's four kernel forms): bit-exact vs the oracle's
    embeddings."""
    rng = np.random.default_rng(sum(lens))
    ids = rng.integers(0, OL.VOCAB, sum(lens)).astype(np.int32)
    offsets = np.concatenate([[0], np.cumsum(lens)])
    got = small_encoder.batch(ids, offsets)
    want = run_oracle(small_model, ids, offsets)
    c = cosines(got, want)
    print(f"lens={lens} min cos {c.min():.7f} max abs {np.abs(got - want).max():.3e}")
    assert c.min() >= COS_MIN
    assert np.abs(got - want).max() <= MAX_ABS
    assert np.array_equal(got, want)
    assert np.allclose(np.linalg.norm(got, axis=1), 1.0, atol=1e-5)


def test_packing_invariance(small_encoder):
    rng = np.random.default_rng(3)
    lens = [10, 200, 33, 1]
    ids = rng.integers(0, OL.VOCAB, sum(lens)).astype(np.int32)
    offsets = np.concatenate([[0], np.cumsum(lens)])
    packed = small_encoder.batch(ids, offsets)
    for s, n in enumerate(lens):
        solo = small_encoder.batch(ids[offsets[s]:offsets[s + 1]], [0, n])
        # Every kernel's result for a sequence is independent of the others
        # in the wave (row-wise GEMMs and norms, sequence-aligned attention
        # tiles), so packing does not change a single bit.
        assert np.array_equal(solo[0], packed[s])


def test_repeatable_and_graph_matches_eager(eg2, small_encoder, small_model):
    rng = np.random.default_rng(4)
    ids = rng.integers(0, OL.VOCAB, 300).astype(np.int32)
    offsets = [0, 100, 300]
    a = small_encoder.batch(ids, offsets)
    b = small_encoder.batch(ids, offsets)
    assert np.array_equal(a, b)
    os.environ["EG2_HIP_GRAPH"] = "0"
    try:
        eager = eg2.Encoder(small_model)
        c = eager.batch(ids, offsets)
        eager.close()
    finally:
        del os.environ["EG2_HIP_GRAPH"]
    assert np.array_equal(a, c)


def test_profile_line_times_every_kernel(eg2, small_model, capfd):
    """EG2_HIP_PROFILE=1 runs the forward eagerly with an event after every
    launch and prints, per batch call, the reference's KFD_PROFILE line
    (src/gemma2_kfd.cpp:346-352) as HIP_PROFILE: tokens, batch, wall_ms and
    command_ms, the summed GPU time of each launch name. The embeddings are
    the graph run's bit for bit; every kernel of the forward has a positive
    time; the per-kernel times add up to less than the wall time (which also
    holds the host staging and copies) and to most of it."""
    import json

    rng = np.random.default_rng(12)
    ids = rng.integers(0, OL.VOCAB, 900).astype(np.int32)
    offsets = [0, 700, 900]  # a wave over 512 tokens: the 2048-key softmax form
    ref = eg2.Encoder(small_model)
    want = ref.batch(ids, offsets)
    ref.close()
    os.environ["EG2_HIP_PROFILE"] = "1"
    try:
        enc = eg2.Encoder(small_model)
        capfd.readouterr()
        got = [enc.batch(ids, offsets) for _ in range(2)]
        enc.close()
    finally:
        del os.environ["EG2_HIP_PROFILE"]
    err = capfd.readouterr().err
    lines = [l for l in err.splitlines() if l.startswith("HIP_PROFILE ")]
    assert len(lines) == 2, err[-2000:]
    for g in got:
        assert np.array_equal(g, want)
    kernels = {"embed", "gemm_qkv_rope", "attention_scores", "attention_softmax", "attention_context", "gemm_o",
               "residual", "gemm_gate_up_geglu", "gemm_down", "output_norm", "pool", "dense_quant", "dense_2",
               "dense_3", "dense_l2"}
    for line in lines:
        rec = json.loads(line[len("HIP_PROFILE "):])
        assert list(rec) == ["tokens", "batch", "wall_ms", "command_ms"]
        assert rec["tokens"] == 900 and rec["batch"] == 2
        ms = rec["command_ms"]
        assert set(ms) == kernels and list(ms) == sorted(ms)
        assert all(v > 0 for v in ms.values()), ms
        total = sum(ms.values())
        print(f"wall {rec['wall_ms']:.3f} ms, kernels {total:.3f} ms: {ms}")
        assert 0.3 * rec["wall_ms"] < total <= rec["wall_ms"]


def test_invalid_batches_fail_without_poisoning(eg2, small_encoder):
    ids = np.zeros(10, np.int32)
    cases = [([0, 5, 5, 10], "offsets"), ([1, 10], "1..2048"), ([0, 0], "offsets")]
    for offsets, msg in cases:
        with pytest.raises(eg2.HipError, match=msg):
            small_encoder.batch(ids, offsets)
    with pytest.raises(eg2.HipError, match="out of range"):
        small_encoder.batch(np.array([0, OL.VOCAB], np.int32), [0, 2])
    with pytest.raises(eg2.HipError, match="1..2048"):
        small_encoder.batch(np.zeros(2049, np.int32), [0, 2049])
    out = small_encoder.batch(ids, [0, 10])  # still usable
    assert np.isfinite(out).all()


def test_injected_hip_failure_poisons_the_context(eg2, small_model):
    """A failing HIP call (forced from the host by the test hook, no device
    fault) makes the call return false with a "HIP:" message, and every later
    call on the context fails until it is recreated (src/gemma2_kfd.cpp:190-191,
    214-215, 270)."""
    enc = eg2.Encoder(small_model)
    try:
        ids = np.arange(40, dtype=np.int32)
        good = enc.batch(ids, [0, 40])
        eg2.lib().eg2_kfd_inject_failure(enc.ctx)
        with pytest.raises(eg2.HipError, match=r"^HIP: .*injected HIP failure"):
            enc.batch(ids, [0, 40])
        for call in (lambda: enc.batch(ids, [0, 40]), lambda: enc.stage(ids, [0, 40], 1),
                     lambda: enc.stream(ids, [0, 40], [768])):
            with pytest.raises(eg2.HipError, match="restart process"):
                call()
    finally:
        enc.close()
    fresh = eg2.Encoder(small_model)
    try:
        assert np.array_equal(fresh.batch(ids, [0, 40]), good)
    finally:
        fresh.close()


def test_env_flags_are_validated(eg2, small_model):
    os.environ["EG2_HIP_GRAPH"] = "yes"
    try:
        with pytest.raises(eg2.HipError, match="EG2_HIP_GRAPH must be 0 or 1"):
            eg2.Encoder(small_model)
    finally:
        del os.environ["EG2_HIP_GRAPH"]


def test_env_lanes(eg2, small_model):
    for bad in ("0", "9", "x", ""):
        os.environ["EG2_HIP_LANES"] = bad
        try:
            with pytest.raises(eg2.HipError, match="EG2_HIP_LANES must be 1..8"):
                eg2.Encoder(small_model)
        finally:
            del os.environ["EG2_HIP_LANES"]
    os.environ["EG2_HIP_LANES"] = "1"
    try:
        one = eg2.Encoder(small_model)
    finally:
        del os.environ["EG2_HIP_LANES"]
    try:
        assert one.lanes == 1
        ids = np.arange(50, dtype=np.int32)
        assert np.isfinite(one.batch(ids, [0, 20, 50])).all()
    finally:
        one.close()
    # default: 4 lanes, each stream on a hardware queue of its own whatever
    # the runtime's queue count (GPU_MAX_HW_QUEUES)
    saved = os.environ.pop("GPU_MAX_HW_QUEUES", None)
    try:
        for queues, want in ((None, 4), ("2", 4), ("4", 4), ("8", 4), ("x", 4)):
            if queues is None:
                os.environ.pop("GPU_MAX_HW_QUEUES", None)
            else:
                os.environ["GPU_MAX_HW_QUEUES"] = queues
            enc = eg2.Encoder(small_model)
            try:
                assert enc.lanes == want, (queues, enc.lanes)
            finally:
                enc.close()
    finally:
        if saved is None:
            os.environ.pop("GPU_MAX_HW_QUEUES", None)
        else:
            os.environ["GPU_MAX_HW_QUEUES"] = saved


def waves_for_lanes(n):
    rng = np.random.default_rng(11)
    out = []
    for i in range(n):
        lens = [[300, 5], [2048], [1, 1, 1, 40], [900, 700, 64], [17]][i % 5]
        out.append((rng.integers(0, OL.VOCAB, sum(lens)).astype(np.int32), np.concatenate([[0], np.cumsum(lens)])))
    return out


def test_lanes_in_flight_match_one_at_a_time(small_encoder):
    """Different waves staged on every lane and launched together (up to
    `lanes` in flight, some twice in a row) give exactly the embeddings each
    wave gets alone."""
    L = small_encoder.lanes
    assert L >= 2
    waves = waves_for_lanes(L)
    alone = [small_encoder.batch(ids, offs) for ids, offs in waves]
    for lane, (ids, offs) in enumerate(waves):
        small_encoder.stage(ids, offs, lane)
    for r in range(2):
        for lane in range(L):
            small_encoder.launch(1 + r, lane)
    for lane in range(L):
        assert np.array_equal(small_encoder.collect(lane), alone[lane])
    # The non-waiting lane query: every lane reports done within the
    # executor's wait limit, and then its collect returns the same result.
    for lane in range(L):
        small_encoder.stage(*waves[lane], lane)
        small_encoder.launch(1, lane)
    t0 = time.monotonic()
    pending = set(range(L))
    while pending and time.monotonic() - t0 < 30:
        pending = {lane for lane in pending if not small_encoder.ready(lane)}
    assert not pending
    for lane in range(L):
        assert small_encoder.ready(lane)
        assert np.array_equal(small_encoder.collect(lane), alone[lane])
    # Restaging a lane whose wave was never collected waits for it first.
    ids, offs = waves[0]
    small_encoder.stage(ids, offs, 1)
    small_encoder.launch(1, 1)
    small_encoder.stage(waves[1][0], waves[1][1], 1)
    small_encoder.launch(1, 1)
    assert np.array_equal(small_encoder.collect(1), alone[1])


def test_concurrent_batch_calls(small_encoder):
    """Threads calling ei_gemma2_kfd_batch at once run on separate lanes;
    every result equals the one-at-a-time result."""
    import threading

    waves = waves_for_lanes(6)
    alone = [small_encoder.batch(ids, offs) for ids, offs in waves]
    errors = []

    def worker(k):
        try:
            for rep in range(3):
                j = (k + rep) % len(waves)
                got = small_encoder.batch(*waves[j])
                if not np.array_equal(got, alone[j]):
                    errors.append((k, rep, j))
        except Exception as e:  # reported below
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(k,)) for k in range(5)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors


def test_full_model_16x128_parity(eg2, gpu, full_model):
    rng = np.random.default_rng(0)
    ids = rng.integers(0, OL.VOCAB, 16 * 128).astype(np.int32)
    offsets = np.arange(0, 16 * 128 + 1, 128)
    enc = eg2.Encoder(full_model)
    try:
        got = enc.batch(ids, offsets)
    finally:
        enc.close()
    want = run_oracle(full_model, ids, offsets)
    c = cosines(got, want)
    print(f"config4 min cos {c.min():.7f} max abs {np.abs(got - want).max():.3e}")
    assert c.min() >= COS_MIN
    assert np.abs(got - want).max() <= MAX_ABS
    assert np.array_equal(got, want)
    # Matryoshka prefixes of the served embedding (kernels.c:398-407).
    for dims in (128, 256, 512):
        a, b = got[:, :dims].copy(), want[:, :dims].copy()
        a /= np.linalg.norm(a, axis=1, keepdims=True)
        b /= np.linalg.norm(b, axis=1, keepdims=True)
        assert cosines(a, b).min() >= COS_MIN
