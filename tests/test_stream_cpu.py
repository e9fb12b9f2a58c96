"""Wave packing (the dynamic batcher's fit rules, inference_service.c:519-681)
and Matryoshka prefix normalisation (kernels.c:393-407), on the CPU."""
import numpy as np
import pytest

from oracle_lib import fptr, oracle


def test_lookahead_packing_worked_example(eg2):
    """budget 10, sequence limit 8, 3 per wave, lookahead (:631-663):
    wave 1 = head 0 (4) + 2 (3) + 4 (2) (1 does not fit, 3 is oversized),
    wave 2 = 1 (7) + 5 (2) + 7 (1) (6 would exceed the budget), then the
    oversized 3 alone and 6; each wave runs longest first."""
    cfg = eg2.batch_config(max_batch_tokens=10, max_batch_sequence_tokens=8, max_batch_requests=3)
    assert eg2.pack_waves([4, 7, 3, 9, 2, 2, 5, 1], cfg) == [[0, 2, 4], [1, 5, 7], [3], [6]]


def test_in_order_packing_worked_example(eg2):
    """Without lookahead (:611-630) a wave takes from the head until the
    first entry that does not fit; ties in the longest-first sort keep
    queue order."""
    cfg = eg2.batch_config(max_batch_tokens=10, max_batch_sequence_tokens=8, max_batch_requests=3, lookahead=0)
    assert eg2.pack_waves([4, 7, 3, 9, 2, 2, 5, 1], cfg) == [[0], [1, 2], [3], [6, 4, 5], [7]]
    unsorted = eg2.batch_config(max_batch_tokens=10, max_batch_sequence_tokens=8, max_batch_requests=3,
                                lookahead=0, sort_longest_first=0)
    assert eg2.pack_waves([4, 7, 3, 9, 2, 2, 5, 1], unsorted) == [[0], [1, 2], [3], [4, 5, 6], [7]]


@pytest.mark.parametrize("fillers,joins", [(15, True), (16, False)])
def test_lookahead_scans_eight_times_the_wave_size(eg2, fillers, joins):
    """The scan behind the head stops after 8 * max_batch_requests entries
    (inference_service.c:415-417): with 2 requests per wave, an entry that
    fits joins only if at most 15 non-fitting entries precede it."""
    cfg = eg2.batch_config(max_batch_tokens=10, max_batch_sequence_tokens=10, max_batch_requests=2)
    lengths = [6] + [5] * fillers + [4]
    first = eg2.pack_waves(lengths, cfg)[0]
    assert first == ([0, fillers + 1] if joins else [0])


def test_packing_properties_on_random_queues(eg2):
    rng = np.random.default_rng(5)
    for trial in range(200):
        cfg = eg2.batch_config(max_batch_tokens=int(rng.integers(8, 64)), max_batch_sequence_tokens=int(rng.integers(4, 64)),
                               max_batch_requests=int(rng.integers(1, 8)), lookahead=int(rng.integers(0, 2)))
        lengths = rng.integers(1, 80, int(rng.integers(1, 60))).tolist()
        waves = eg2.pack_waves(lengths, cfg)
        flat = [i for w in waves for i in w]
        assert sorted(flat) == list(range(len(lengths)))  # every sequence exactly once
        placed = set()
        for w in waves:
            head = min(i for i in range(len(lengths)) if i not in placed)
            assert head in w  # the queue head always leads a wave
            assert len(w) <= cfg.max_batch_requests
            lens = [lengths[i] for i in w]
            assert lens == sorted(lens, reverse=True)
            if len(w) > 1:
                assert sum(lens) <= cfg.max_batch_tokens and max(lens) <= cfg.max_batch_sequence_tokens
            ties = [i for i in w]
            for a, b in zip(ties, ties[1:]):
                if lengths[a] == lengths[b]:
                    assert a < b  # equal lengths keep queue order
            placed.update(w)


def test_packing_rejects_bad_arguments(eg2):
    with pytest.raises(eg2.HipError):
        eg2.pack_waves([3, 0, 2])
    with pytest.raises(eg2.HipError):
        eg2.pack_waves([3], eg2.batch_config(max_batch_requests=0))
    assert eg2.pack_waves([]) == []


@pytest.mark.parametrize("dims", [128, 256, 512, 768])
def test_prefix_normalisation_matches_oracle(eg2, dims):
    rng = np.random.default_rng(dims)
    for _ in range(20):
        e = (rng.standard_normal(768) * 10.0 ** rng.uniform(-3, 3)).astype(np.float32)
        want = e.copy()
        assert oracle().or_normalize_prefix(fptr(want), dims) == 1
        assert np.array_equal(eg2.normalize_prefix(e, dims), want)
    with pytest.raises(eg2.HipError):
        eg2.normalize_prefix(np.ones(768, np.float32), 100)
