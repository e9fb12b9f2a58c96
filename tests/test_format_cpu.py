"""The output side of the path (include/eg2_format.h): float text, base64
and the embedding response body.

Float text is pinned by the reference's own float_format.c: byte-exact
against tests/golden/float_text.npz (its outputs over specials, binade edges,
subnormals, powers of ten, random bit patterns and embedding-like values),
against the compiled reference over a strided sweep of all bit patterns
where that is built, and by what the definition fixes: every text reads
back as the same float, and no shorter digit string does."""
import base64
import ctypes as C
import ctypes.util
import json
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden", "float_text.npz")
LIBC = C.CDLL(ctypes.util.find_library("c"))
LIBC.strtof.restype = C.c_float
LIBC.strtof.argtypes = [C.c_char_p, C.POINTER(C.c_char_p)]


def bits_of(x):
    return int(np.float32(x).view(np.uint32))


def reads_back(text, value):
    return bits_of(LIBC.strtof(text.encode(), None)) == bits_of(value)


def test_matches_reference_vectors(eg2):
    g = np.load(GOLDEN)
    text, offs = g["text"].tobytes(), g["offsets"]
    bad = []
    for i, b in enumerate(g["bits"]):
        want = text[offs[i]:offs[i + 1]].decode()
        got = eg2.f32_to_chars(np.uint32(b).view(np.float32))
        if got != want:
            bad.append((hex(int(b)), want, got))
    assert not bad, bad[:5]
    assert len(g["bits"]) > 20000


def test_layout_examples(eg2):
    cases = [(0.0, "0.0"), (-0.0, "-0.0"), (1.0, "1.0"), (100.0, "100.0"), (123456.0, "123456.0"),
             (1234567.0, "1.234567e+06"), (1e7, "1e+07"), (0.5, "0.5"), (0.001, "0.001"), (0.0001, "0.0001"),
             (0.00001, "1e-05"), (1.5e-5, "1.5e-05"), (-2.5, "-2.5"), (3.4028234663852886e38, "3.4028235e+38"),
             (1e-45, "1e-45"), (0.1, "0.1"), (1.0 / 3.0, "0.33333334")]
    for v, want in cases:
        assert eg2.f32_to_chars(np.float32(v)) == want, v
    assert eg2.f32_to_chars(np.float32(np.inf)) is None
    assert eg2.f32_to_chars(np.float32(np.nan)) is None


def test_round_trip_and_shortest(eg2):
    """Every text reads back exactly; dropping one digit (rounding the digit
    string down or up) never does."""
    rng = np.random.default_rng(7)
    vals = np.concatenate([rng.integers(0, 2 ** 32, 3000, dtype=np.uint64).astype(np.uint32).view(np.float32),
                           (rng.standard_normal(3000) / 30).astype(np.float32)])
    for v in vals[np.isfinite(vals)]:
        t = eg2.f32_to_chars(v)
        assert reads_back(t, v), (v, t)
        mant, _, exp = t.lstrip("-").partition("e")
        digits = mant.replace(".", "").lstrip("0")
        if len(digits.rstrip("0")) <= 1:
            continue
        # shortest: no (len - 1)-digit decimal reads back as v
        sci = f"{abs(float(v)):.{len(digits.rstrip('0')) - 1}e}"
        lead, ex = sci.split("e")
        d = int(lead.replace(".", "")) // 10
        p = len(lead.replace(".", "")) - 1
        for cand in (d, d + 1):
            txt = f"{cand}e{int(ex) - p + 1}"
            assert not reads_back(("-" if t.startswith("-") else "") + txt, v), (v, t, txt)


def test_strided_sweep_against_reference():
    """Every 65,537th float bit pattern against the compiled reference
    (oracle/float_text_check.c), where oracle/_ref is built."""
    check = os.path.join(ROOT, "oracle", "_ref", "float_text_check")
    ref_so = os.path.join(ROOT, "oracle", "_ref", "libref.so")
    if not (os.path.exists(check) and os.path.exists(ref_so)):
        pytest.skip("oracle/_ref is not built (no reference tree)")
    ours = os.path.join(ROOT, "embeddinggemma2-amdkfd_amd", "libeg2hip.so")
    out = subprocess.run([check, "65537", "4", ref_so, ours], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "0 mismatches" in out.stdout


def test_base64_is_the_little_endian_bytes(eg2):
    rng = np.random.default_rng(3)
    for n in (1, 2, 3, 128, 767, 768):
        v = rng.standard_normal(n).astype(np.float32)
        assert eg2.base64_f32(v) == base64.b64encode(v.astype("<f4").tobytes()).decode()


def normalised(eg2, e, dims):
    return np.stack([eg2.normalize_prefix(row, dims) for row in e])


@pytest.mark.parametrize("dims", [128, 768])
def test_response_bodies(eg2, dims):
    rng = np.random.default_rng(dims)
    e = rng.standard_normal((3, 768)).astype(np.float32)
    e /= np.linalg.norm(e, axis=1, keepdims=True)
    n = normalised(eg2, e, dims)
    arrays = ["[" + ",".join(eg2.f32_to_chars(x) for x in row[:dims]) + "]" for row in n]
    body = eg2.embeddings_response(e, dims)
    assert body == '{"embeddings":[' + ",".join(arrays) + "]}"
    assert np.array_equal(np.array(json.loads(body)["embeddings"], np.float32), n[:, :dims])
    model = 'emb"gemma\\\n\x01'
    body = eg2.embeddings_response(e, dims, api="openai", encoding="base64", model=model, prompt_tokens=42)
    items = ",".join('{"object":"embedding","embedding":"' + eg2.base64_f32(row[:dims]) + f'","index":{i}}}'
                     for i, row in enumerate(n))
    assert body == ('{"object":"list","data":[' + items + '],"model":"emb\\"gemma\\\\\\n\\u0001",'
                    '"usage":{"prompt_tokens":42,"total_tokens":42}}')
    j = json.loads(body)
    assert j["model"] == model
    got = np.stack([np.frombuffer(base64.b64decode(d["embedding"]), "<f4") for d in j["data"]])
    assert np.array_equal(got, n[:, :dims])


def test_response_rejects_bad_input(eg2):
    e = np.ones((1, 768), np.float32)
    with pytest.raises(ValueError):
        eg2.embeddings_response(e, 300)
    e[0, 5] = np.nan
    with pytest.raises(ValueError):
        eg2.embeddings_response(e, 768)
