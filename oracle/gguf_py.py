"""Independent GGUF v3 reader in numpy (oracle-side infrastructure): turns a
synthetic gemma-embedding file into the oracle's model dict, so the oracle
never goes through the product's own C++ reader."""
import struct

import numpy as np

from oracle_lib import Q8

_SCALAR = {0: "<u1", 1: "<i1", 2: "<u2", 3: "<i2", 4: "<u4", 5: "<i4", 6: "<f4", 7: "<u1", 10: "<u8", 11: "<i8",
           12: "<f8"}


def read(path):
    buf = np.memmap(path, dtype=np.uint8, mode="r")
    b = bytes(buf[: min(len(buf), 1 << 20)])
    pos = 0

    def take(fmt):
        nonlocal pos
        v = struct.unpack_from(fmt, b, pos)
        pos += struct.calcsize(fmt)
        return v[0] if len(v) == 1 else v

    def string():
        n = take("<Q")
        nonlocal pos
        s = b[pos:pos + n].decode()
        pos += n
        return s

    assert take("<I") == 0x46554747
    assert take("<I") == 3
    n_t, n_kv = take("<Q"), take("<Q")
    kvs = {}
    for _ in range(n_kv):
        key = string()
        ty = take("<I")
        if ty == 8:
            kvs[key] = string()
        elif ty == 9:
            raise NotImplementedError("arrays are not written by the synthetic model")
        else:
            dt = np.dtype(_SCALAR[ty])
            kvs[key] = np.frombuffer(b, dtype=dt, count=1, offset=pos)[0].item()
            pos += dt.itemsize
    infos = []
    for _ in range(n_t):
        name = string()
        nd = take("<I")
        ne = [take("<Q") for _ in range(nd)]
        ty, off = take("<I"), take("<Q")
        infos.append((name, ne, ty, off))
    align = kvs.get("general.alignment", 32)
    data_off = (pos + align - 1) // align * align
    tensors = {}
    for name, ne, ty, off in infos:
        start = data_off + off
        if ty == 8:
            rows = int(np.prod(ne[1:])) if len(ne) > 1 else 1
            n = rows * ne[0] // 32
            arr = np.frombuffer(buf, dtype=Q8, count=n, offset=start).reshape(rows, ne[0] // 32)
        elif ty == 0:
            arr = np.frombuffer(buf, dtype=np.float32, count=int(np.prod(ne)), offset=start)
        else:
            raise NotImplementedError(ty)
        tensors[name] = (ty, ne, arr)
    return kvs, tensors


def oracle_model(path):
    """Model dict for oracle_lib.forward from a gemma-embedding GGUF."""
    kvs, t = read(path)
    n_layer = kvs["gemma-embedding.block_count"]
    period = kvs.get("gemma-embedding.attention.sliding_window_pattern", 6)
    window = kvs.get("gemma-embedding.attention.sliding_window", 512)
    base_full = kvs.get("gemma-embedding.rope.freq_base", 1e6)
    base_swa = kvs.get("gemma-embedding.rope.freq_base_swa", 1e4)
    layers = []
    for il in range(n_layer):
        p = f"blk.{il}."
        swa = (il % period) < (period - 1)
        L = {n: np.ascontiguousarray(t[p + n + ".weight"][2]) for n in (
            "attn_q", "attn_k", "attn_v", "attn_output", "ffn_up", "ffn_gate", "ffn_down", "attn_norm",
            "attn_q_norm", "attn_k_norm", "post_attention_norm", "ffn_norm", "post_ffw_norm")}
        L["rope_base"] = float(np.float32(base_swa if swa else base_full))
        L["window"] = int(window) if swa else 0
        layers.append(L)
    m = dict(token_embd=t["token_embd.weight"][2], output_norm=np.ascontiguousarray(t["output_norm.weight"][2]),
             layers=layers, eps=float(np.float32(kvs.get("gemma-embedding.attention.layer_norm_rms_epsilon", 1e-6))))
    if "dense_2.weight" in t:
        m["dense_2"] = np.ascontiguousarray(t["dense_2.weight"][2])
        m["dense_3"] = np.ascontiguousarray(t["dense_3.weight"][2])
    return m


def write_kv(path, kvs):
    """GGUF v3 file holding key-values only (no tensors), for the tokenizer's
    keys. kvs: (key, kind, value) with kind 'str', 'u32', 'bool', 'arr_str'
    (list of bytes), 'arr_f32' or 'arr_i32'."""
    out = [struct.pack("<IIQQ", 0x46554747, 3, 0, len(kvs))]

    def s(b):
        b = b.encode() if isinstance(b, str) else bytes(b)
        return struct.pack("<Q", len(b)) + b

    for key, kind, val in kvs:
        out.append(s(key))
        if kind == "str":
            out.append(struct.pack("<I", 8) + s(val))
        elif kind == "u32":
            out.append(struct.pack("<II", 4, int(val)))
        elif kind == "bool":
            out.append(struct.pack("<IB", 7, 1 if val else 0))
        elif kind == "arr_str":
            out.append(struct.pack("<IIQ", 9, 8, len(val)) + b"".join(s(v) for v in val))
        elif kind == "arr_f32":
            a = np.ascontiguousarray(val, dtype="<f4")
            out.append(struct.pack("<IIQ", 9, 6, a.size) + a.tobytes())
        elif kind == "arr_i32":
            a = np.ascontiguousarray(val, dtype="<i4")
            out.append(struct.pack("<IIQ", 9, 5, a.size) + a.tobytes())
        else:
            raise ValueError(kind)
    blob = b"".join(out)
    blob += b"\0" * ((-len(blob)) % 32)
    with open(path, "wb") as f:
        f.write(blob)
