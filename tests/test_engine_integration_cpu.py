"""The reference's own engine, built against this library (CPU only).

The executor boundary claims that the reference's engine drops onto
libeg2hip.so with three engine edits (apply_integration_edits below: a
Q8_0 `gemma-embedding` file routed to the kfd executor). This test builds that:
it copies the engine's C sources from the reference tree (present only in
the build container; the test is skipped elsewhere) into a temporary
directory, applies those edits there, compiles them with EI_ENABLE_KFD=1
against this repository's include/ and links libeg2hip.so. A probe program
then calls the engine's ei_engine_load_backend(..., "kfd") on a synthetic
24-layer Q8_0 gemma-embedding GGUF with a 262,144-piece vocabulary, in a
subprocess. With no GPU here, the library's create validates every tensor
of the engine's parsed file and then stops at the device check, so the
engine dies with "HIP: supported HIP device not found": the engine's
routing reached this library with a model it accepted. A model whose
dense_2 tensor has the wrong type (a tensor the engine's loader does not
read) dies in the library's validation instead, before any device call."""
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_SRC = "/root/reference/vendor/embeddinggemma.c/src"
SOURCES = ["engine.c", "model.c", "gguf.c", "tokenizer.c", "quants.c", "kernels.c", "parallel.c", "gemma2.c",
           "gemma2_fast.c", "gemma2_fast_x86.c"]
HEADERS = ["engine.h", "model.h", "gguf.h", "tokenizer.h", "quants.h", "kernels.h", "parallel.h", "gemma2.h",
           "gemma2_fast_x86.h", "common.h"]
VOCAB = 262144

pytestmark = pytest.mark.skipif(not os.path.exists(os.path.join(REF_SRC, "engine.c")) or not shutil.which("gcc"),
                                reason="the reference engine sources (build container only) or gcc are absent")


def edit(path, old, new, count=1):
    s = open(path).read()
    assert s.count(old) == count, (path, old)
    open(path, "w").write(s.replace(old, new))


def apply_integration_edits(d):
    """The three engine edits that route a Q8_0 gemma-embedding file to the
    kfd executor: a q8_matrices flag in the model, the layer matrices typed
    after the first layer's attention weight (Q8_0 or Q4_0), and the engine
    creating the kfd executor when that backend is asked for."""
    edit(os.path.join(d, "model.h"), "    bool embeddinggemma2;\n",
         "    bool embeddinggemma2;\n    bool q8_matrices;\n")
    model_c = os.path.join(d, "model.c")
    edit(model_c, "        for (int il = 0; il < EI_N_LAYER; il++) {\n",
         "        const ei_tensor *probe = ei_gguf_tensor(g, \"blk.0.attn_q.weight\", true);\n"
         "        const uint32_t mt = probe->type == EI_T_Q8_0 ? EI_T_Q8_0 : EI_T_Q4_0;\n"
         "        m->q8_matrices = mt == EI_T_Q8_0;\n"
         "        for (int il = 0; il < EI_N_LAYER; il++) {\n")
    for name in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_up", "ffn_gate", "ffn_down"):
        s = open(model_c).read()
        i = s.index(f"T({name},")
        j = s.index("EI_T_Q4_0", i)
        assert j - i < 60
        open(model_c, "w").write(s[:j] + "mt       " + s[j + len("EI_T_Q4_0"):])
    engine_c = os.path.join(d, "engine.c")
    edit(engine_c, "    e->backend_name = \"cpu\";\n    if (e->model.embeddinggemma2) {\n",
         "    e->backend_name = \"cpu\";\n"
         "#if defined(EI_ENABLE_KFD)\n"
         "    if (!e->model.embeddinggemma2 && backend && !strcmp(backend, \"kfd\")) {\n"
         "        char err[512];\n"
         "        e->gemma2_kfd = ei_gemma2_kfd_create(&e->model.gguf, err, sizeof err);\n"
         "        if (!e->gemma2_kfd) ei_die(\"%s\", err);\n"
         "        e->backend_name = \"kfd\";\n"
         "        return;\n"
         "    }\n"
         "#endif\n"
         "    if (e->model.q8_matrices) ei_die(\"Q8_0 gemma-embedding matrices need --backend kfd\");\n"
         "    if (e->model.embeddinggemma2) {\n")
    edit(engine_c, "    if (!e->model.embeddinggemma2) ensure_workspace(e, total_tokens);\n",
         "    if (!e->model.embeddinggemma2 && !e->gemma2_kfd) ensure_workspace(e, total_tokens);\n")


PROBE = r"""
#include <stdio.h>
#include "engine.h"
int main(int argc, char **argv) {
    ei_engine e;
    ei_engine_load_backend(&e, argv[1], argv[2]);
    printf("backend %s\n", e.backend_name);
    ei_engine_free(&e);
    return 0;
}
"""


def with_vocabulary(src, dst, q4_dense_2=False):
    """dst = the GGUF src (as the library's synthetic writer made it) with
    the tokenizer arrays the engine's loader requires added to its
    key-values (tensor data offsets are relative to the data section, so
    the tensors are copied unchanged)."""
    with open(src, "rb") as f:
        head = f.read(1 << 20)
    magic, version, n_t, n_kv = struct.unpack_from("<IIQQ", head, 0)
    assert magic == 0x46554747 and version == 3
    pos = 24

    def skip_str(p):
        n = struct.unpack_from("<Q", head, p)[0]
        return p + 8 + n

    kv_start = pos
    align = 32
    for _ in range(n_kv):
        key_end = skip_str(pos)
        key = head[pos + 8:key_end].decode()
        ty = struct.unpack_from("<I", head, key_end)[0]
        pos = key_end + 4
        if ty == 8:
            pos = skip_str(pos)
        else:
            size = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}[ty]
            if key == "general.alignment":
                align = struct.unpack_from("<I", head, pos)[0]
            pos += size
    kv_bytes = head[kv_start:pos]
    info_start = pos
    infos = []
    for _ in range(n_t):
        name_end = skip_str(pos)
        nd = struct.unpack_from("<I", head, name_end)[0]
        p = name_end + 4 + 8 * nd
        infos.append((head[pos + 8:name_end].decode(), p))  # p: offset of the type field
        pos = p + 4 + 8
    info_bytes = bytearray(head[info_start:pos])
    if q4_dense_2:  # a type the engine's loader does not check and the library's validation rejects
        for name, p in infos:
            if name == "dense_2.weight":
                struct.pack_into("<I", info_bytes, p - info_start, 2)  # GGML Q4_0
    data_off = (pos + align - 1) // align * align

    def s(b):
        b = b.encode() if isinstance(b, str) else b
        return struct.pack("<Q", len(b)) + b

    pieces = [b"<pad>", b"<eos>", b"<bos>", b"<unk>"] + [b"<0x%02X>" % i for i in range(256)]
    pieces += [b"\xe2\x96\x81t%d" % i for i in range(VOCAB - len(pieces))]
    types = np.ones(VOCAB, "<i4")
    types[:4] = 3
    types[4:260] = 6
    extra = [s("tokenizer.ggml.tokens") + struct.pack("<IIQ", 9, 8, VOCAB) + b"".join(s(p) for p in pieces),
             s("tokenizer.ggml.scores") + struct.pack("<IIQ", 9, 6, VOCAB) +
             (-np.arange(VOCAB, dtype="<f4")).tobytes(),
             s("tokenizer.ggml.token_type") + struct.pack("<IIQ", 9, 5, VOCAB) + types.tobytes()]
    header = struct.pack("<IIQQ", magic, version, n_t, n_kv + len(extra)) + kv_bytes + b"".join(extra) + info_bytes
    header += b"\0" * ((-len(header)) % align)
    with open(src, "rb") as f, open(dst, "wb") as out:
        out.write(header)
        f.seek(data_off)
        shutil.copyfileobj(f, out, 1 << 24)


@pytest.fixture(scope="module")
def engine_probe(tmp_path_factory):
    lib = os.path.join(ROOT, "embeddinggemma2-amdkfd_amd", "libeg2hip.so")
    if not os.path.exists(lib):
        pytest.skip("libeg2hip.so is not built")
    d = str(tmp_path_factory.mktemp("engine"))
    for f in SOURCES + HEADERS:
        shutil.copy(os.path.join(REF_SRC, f), d)
    apply_integration_edits(d)
    with open(os.path.join(d, "probe.c"), "w") as f:
        f.write(PROBE)
    exe = os.path.join(d, "engine_probe")
    cmd = ["gcc", "-O1", "-DEI_ENABLE_KFD=1", "-I" + d, "-I" + os.path.join(ROOT, "include"), "-o", exe,
           os.path.join(d, "probe.c")] + [os.path.join(d, f) for f in SOURCES] + [
           lib, "-Wl,-rpath," + os.path.dirname(lib), "-lm", "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-4000:]
    return exe


@pytest.fixture(scope="module")
def q8_model(eg2, tmp_path_factory):
    d = tmp_path_factory.mktemp("model")
    raw = str(d / "raw.gguf")
    eg2.synth_gguf(raw, seed=5, n_layer=24, dense_head=True, threads=8)
    good, bad = str(d / "q8.gguf"), str(d / "q8_bad.gguf")
    with_vocabulary(raw, good)
    with_vocabulary(raw, bad, q4_dense_2=True)
    os.remove(raw)
    return good, bad


def run_probe(exe, model, backend):
    env = dict(os.environ, HIP_VISIBLE_DEVICES="", ROCR_VISIBLE_DEVICES="")
    return subprocess.run([exe, model, backend], capture_output=True, text=True, timeout=600, env=env)


def test_reference_engine_routes_a_q8_model_to_this_library(engine_probe, q8_model):
    r = run_probe(engine_probe, q8_model[0], "kfd")
    print(r.stdout[-500:], r.stderr[-500:])
    assert r.returncode != 0
    assert "HIP: supported HIP device not found" in r.stderr, r.stderr[-2000:]


def test_reference_engine_reports_the_librarys_validation(engine_probe, q8_model):
    r = run_probe(engine_probe, q8_model[1], "kfd")
    assert r.returncode != 0
    assert "HIP: unexpected type: dense_2.weight" in r.stderr, r.stderr[-2000:]
    assert "device not found" not in r.stderr


def test_reference_engine_keeps_q8_files_off_its_cpu_path(engine_probe, q8_model):
    r = run_probe(engine_probe, q8_model[0], "cpu")
    assert r.returncode != 0
    assert "Q8_0 gemma-embedding matrices need --backend kfd" in r.stderr, r.stderr[-2000:]
