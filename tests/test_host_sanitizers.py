"""The library's host code and the CPU oracle under AddressSanitizer +
UndefinedBehaviorSanitizer and under ThreadSanitizer.

tests/host_sanitize/Makefile builds every source of libeg2hip with the
sanitizer on the host pass only (the device code is built as usual), plus
the oracle, and links them with host_check.cpp, which runs the host-side
parts without a GPU: the executor's model validation (including corrupted
tensor records), the attention plan builder on random packings with
exact-size buffers, the Q8_0 row-tile repacking, the wave packer, the
float-text / base64 / response formatting, the GGUF reader on truncated
files, the threaded synthetic-model writer, the tokenizer (single and
threaded batch forms) and the oracle's threaded GEMM and encoder layer. A
sanitizer finding aborts the run. The tokenizer's ids are also compared
with the reference's ids of the golden fixture."""
import os
import shutil
import subprocess

import numpy as np
import pytest

from test_tokenizer_cpu import GOLDEN, make_tokenizer_file, unblob

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN_DIR = os.path.join(ROOT, "tests", "host_sanitize")

pytestmark = pytest.mark.skipif(shutil.which("make") is None or not os.path.exists("/opt/rocm/bin/hipcc"),
                                reason="needs make and hipcc")


def build(target):
    jobs = str(min(8, os.cpu_count() or 2))
    subprocess.run(["make", "-s", "-j", jobs, target], cwd=SAN_DIR, check=True, capture_output=True, timeout=900)
    return os.path.join(SAN_DIR, "_build", target, "host_check")


def run_check(exe, tmp_path, env_extra):
    g = np.load(GOLDEN)
    make_tokenizer_file(g, "spm", str(tmp_path / "tok.gguf"))
    texts = unblob(g["text"], g["text_offsets"])[:120]
    offs = np.concatenate([[0], np.cumsum([len(t) for t in texts])]).astype(np.uint64)
    with open(tmp_path / "texts.bin", "wb") as f:
        f.write(np.uint64(len(texts)).tobytes() + offs.tobytes() + b"".join(texts))
    env = dict(os.environ, **env_extra)
    r = subprocess.run([exe, str(tmp_path)], capture_output=True, text=True, timeout=900, env=env)
    assert r.returncode == 0 and "host checks passed" in r.stdout, r.stdout[-2000:] + r.stderr[-6000:]
    raw = open(tmp_path / "ids.bin", "rb").read()
    n = int(np.frombuffer(raw[:8], np.uint64)[0])
    id_offs = np.frombuffer(raw[8:8 + 8 * (n + 1)], np.uint64)
    ids = np.frombuffer(raw[8 + 8 * (n + 1):], np.int32)
    want_ids, want_offs = g["spm_ids"], g["spm_id_offsets"]
    # the fixture lists each text under four (add_special, parse_special)
    # pairs; (1, 1) is the second
    for i in range(n):
        k = 4 * i + 1
        want = want_ids[want_offs[k]:want_offs[k + 1]]
        assert np.array_equal(ids[id_offs[i]:id_offs[i + 1]], want), i


def test_host_code_under_address_and_undefined_behaviour_sanitizers(tmp_path):
    exe = build("asan")
    run_check(exe, tmp_path, {"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=1:strict_string_checks=1",
                              "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"})


def test_host_code_under_thread_sanitizer(tmp_path):
    exe = build("tsan")
    run_check(exe, tmp_path, {"TSAN_OPTIONS": "halt_on_error=1:second_deadlock_stack=1"})
