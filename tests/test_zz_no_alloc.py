"""The allocation-free attention entry point (eg2_hip_attention_static: plan
built on the device, plan and scores in the library's static per-device
array) against eg2_hip_attention with a host-built plan and a caller-owned
scores buffer: bit-identical context values and scales, on two calls in a
row (the second smaller, so the first call's plan and scores are still in
the array), for full and windowed attention; and its limits rejected on
the host before anything is launched."""
import ctypes as C

import numpy as np
import pytest

from oracle_lib import N_EMBD

pytestmark = pytest.mark.gpu


def _packing(rng, total, segments, lo=8, hi=512):
    """Lengths log-uniform in [lo, hi], scaled to sum to `total`."""
    raw = np.exp(rng.uniform(np.log(lo), np.log(hi), segments))
    lens = np.maximum(1, np.floor(raw / raw.sum() * total)).astype(np.int64)
    lens[-1] += total - lens.sum()
    assert lens.min() >= 1 and lens.sum() == total
    return np.concatenate([[0], np.cumsum(lens)])


def _qkv(rng, rows):
    a = rng.standard_normal((rows, 1280)).astype(np.float32)
    a[:, :768] *= np.float32(1.0 / 16.0)
    return a


def _run_both(eg2, gpu, qkv_h, offsets, window):
    import torch

    rows = qkv_h.shape[0]
    qkv = torch.from_numpy(qkv_h).to(gpu)
    nq = eg2.q8_tile_bytes(rows, N_EMBD)
    ref_q = torch.zeros(nq, dtype=torch.int8, device=gpu)
    ref_d = torch.zeros((24, rows), dtype=torch.float32, device=gpu)
    plan = eg2.AttentionPlan(list(offsets), gpu, rows)
    eg2.ops.attention_planned(qkv, plan, window, ref_q, ref_d)
    # Outputs start as garbage, so a value the kernels did not write shows.
    out_q = torch.full((nq,), 77, dtype=torch.int8, device=gpu)
    out_d = torch.full((24, rows), float("nan"), dtype=torch.float32, device=gpu)
    offs = torch.from_numpy(np.asarray(offsets, np.int32)).to(gpu)
    eg2.ops.attention_static(qkv, offs, window, out_q, out_d)
    torch.cuda.synchronize()
    # The row tiles hold rows rounded up to 32; only the `rows` rows are outputs.
    unpack = lambda t: eg2.q8_unpack_rows(t.cpu().numpy(), rows, N_EMBD)  # noqa: E731
    return unpack(ref_q), ref_d.cpu().numpy(), unpack(out_q), out_d.cpu().numpy()


def _assert_same(ref_q, ref_d, out_q, out_d):
    assert np.array_equal(ref_q, out_q)
    assert np.array_equal(ref_d.view(np.uint32), out_d.view(np.uint32))


@pytest.mark.parametrize("window", [0, 512])
def test_static_attention_equals_planned_on_two_calls(eg2, gpu, window):
    rng = np.random.default_rng(20 + window)
    # Call 1: 2048 rows, the attention benchmark's packing (16 log-uniform
    # segments in [8, 512]) -- the largest the static array takes.
    offs1 = _packing(rng, 2048, 16)
    print(f"static attention call 1: rows 2048, 16 sequences, window {window}", flush=True)
    _assert_same(*_run_both(eg2, gpu, _qkv(rng, 2048), offs1, window))
    # Call 2, smaller: 301 tokens in 5 sequences plus a 3-row padding
    # sequence (rows a multiple of 4), one of them a single token.
    offs2 = np.array([0, 1, 120, 190, 260, 301, 304])
    print(f"static attention call 2: rows 304, 6 sequences, window {window}", flush=True)
    _assert_same(*_run_both(eg2, gpu, _qkv(rng, 304), offs2, window))


def test_static_attention_one_long_sequence(eg2, gpu):
    """A single 2048-token sequence: the most score floats (3 x 2048^2) the
    static array holds."""
    rng = np.random.default_rng(7)
    print("static attention: one 2048-token sequence", flush=True)
    _assert_same(*_run_both(eg2, gpu, _qkv(rng, 2048), [0, 2048], 0))


def test_static_attention_rejects_sizes_beyond_its_array(eg2, gpu):
    import torch

    rows = 2052
    qkv = torch.zeros((rows, 1280), dtype=torch.float32, device=gpu)
    offs = torch.tensor([0, rows], dtype=torch.int32, device=gpu)
    cq = torch.zeros(eg2.q8_tile_bytes(rows, N_EMBD), dtype=torch.int8, device=gpu)
    cd = torch.zeros((24, rows), dtype=torch.float32, device=gpu)
    with pytest.raises(ValueError, match="static scratch"):
        eg2.ops.attention_static(qkv, offs, 0, cq, cd)
    p = lambda t: C.c_void_p(t.data_ptr())  # noqa: E731
    lib, s = eg2.lib(), C.c_void_p(torch.cuda.current_stream().cuda_stream)
    invalid = 1  # hipErrorInvalidValue
    assert lib.eg2_hip_attention_static(p(qkv), p(offs), 1, 0, rows, p(cq), p(cd), s) == invalid
    assert lib.eg2_hip_attention_static(p(qkv), p(offs), 2049, 0, 2048, p(cq), p(cd), s) == invalid
    assert lib.eg2_hip_attention_static(p(qkv), p(offs), 1, 0, 2046, p(cq), p(cd), s) == invalid
    assert lib.eg2_hip_attention_static(p(qkv), p(offs), 0, 0, 2048, p(cq), p(cd), s) == invalid
    torch.cuda.synchronize()
    assert not cq.any() and not cd.any()  # nothing was launched
